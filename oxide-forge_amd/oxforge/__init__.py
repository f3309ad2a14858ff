"""oxforge -- Python plumbing over the MI355X-native OxideForge compute core.

Everything here calls the C ABI of include/oxforge.h through ctypes
(liboxforge.so + the gfx950 code object).  Device memory is owned by the
library's runtime (its exact-size pool), host data moves with the ABI's copy
calls; nothing here computes on the host.
"""
from __future__ import annotations

import ctypes
import weakref
from ctypes import byref, c_int, c_size_t, c_void_p

import numpy as np

from . import _lib
from ._lib import (ACT_GELU, ACT_IDENTITY, ACT_RELU, ACT_SILU, ADD, DIV, MAP_ADD,  # noqa: F401
                   MAP_EXP_SHIFT, MAP_GELU, MAP_GELU_D, MAP_HALF_SQ, MAP_IDENTITY, MAP_RELU,
                   MAP_RELU_D, MAP_SCALE, MAP_SILU, MAP_SILU_D, MUL, NULL_SLICE, SUB,
                   ForgeError, GemmEpilogue, Slice, call, load)

__all__ = ["Runtime", "DeviceArray", "ForgeError", "device_count", "load"]


def device_count() -> int:
    n = c_int(0)
    call("forge_device_count", byref(n))
    return n.value


class DeviceArray:
    """A device buffer from the runtime pool with a row-major f32 shape."""

    def __init__(self, rt: "Runtime", sl: Slice, shape):
        self.rt = rt
        self.slice = sl
        self.shape = tuple(int(s) for s in shape)

    @property
    def size(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    @property
    def ptr(self) -> int:
        return self.slice.ptr or 0

    def view(self, offset: int, shape) -> "DeviceArray":
        """A sub-range of this buffer (no copy), like DeviceSpan::from_buffer."""
        n = 1
        for s in shape:
            n *= int(s)
        if offset < 0 or offset + n > self.slice.len:
            raise ValueError("view exceeds its buffer")
        sl = Slice((self.slice.ptr or 0) + 4 * offset, n)
        return DeviceArray(self.rt, sl, shape)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=np.float32)
        if self.size:
            call("forge_memcpy_d2h", self.rt.handle, out.ctypes.data_as(c_void_p), self.slice,
                 self.size)
        return out

    def upload(self, host: np.ndarray) -> "DeviceArray":
        host = np.ascontiguousarray(host, dtype=np.float32)
        if host.size != self.size:
            raise ValueError(f"upload of {host.size} elements into {self.size}")
        if host.size:
            call("forge_memcpy_h2d", self.rt.handle, self.slice, host.ctypes.data_as(c_void_p),
                 host.size)
        return self

    def recycle(self) -> None:
        if self.slice.ptr:
            call("forge_recycle", self.rt.handle, self.slice)
            self.slice = Slice(None, 0)


def _sl(a) -> Slice:
    if a is None:
        return NULL_SLICE
    return a.slice


def _epilogue(alpha=1.0, bias=None, residual=None, aux_mul=None, pre_out=None,
              activation=ACT_IDENTITY, update=False, update_scale=0.0, aux_activation=0,
              row_parts_in=None, row_parts=0, row_n=0, row_eps=1e-5, row_div=0,
              row_sumsq_out=None, col_sums_out=None, col_sums_param=None, col_sums_lr=0.0,
              row_sub=None):
    return GemmEpilogue(alpha, _sl(bias), _sl(residual), _sl(aux_mul), _sl(pre_out), activation,
                        1 if update else 0, update_scale, aux_activation, _sl(row_parts_in),
                        row_parts, row_n, row_eps, row_div, _sl(row_sumsq_out), _sl(col_sums_out),
                        _sl(col_sums_param), col_sums_lr, _sl(row_sub))


class Runtime:
    """forge_runtime: CudaRuntime (runtime.rs:34-45) behind the C ABI."""

    def __init__(self, device: int = 0, module_path: str | None = None):
        self.lib = load()
        h = c_void_p()
        path = module_path.encode() if module_path else None
        call("forge_runtime_create", device, path, byref(h))
        self.handle = h
        # Objects built on this runtime (executor models) are closed first.
        self._children = weakref.WeakSet()

    def adopt(self, child) -> None:
        self._children.add(child)

    def close(self) -> None:
        if self.handle:
            for child in list(self._children):
                child.close()
            call("forge_runtime_destroy", self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- device info / sync / streams
    def props(self) -> dict:
        cu, lds, clk = c_int(), c_size_t(), c_int()
        arch = ctypes.create_string_buffer(256)
        call("forge_device_props", self.handle, byref(cu), byref(lds), byref(clk), arch, 256)
        return {"cu_count": cu.value, "lds_bytes": lds.value, "clock_khz": clk.value,
                "arch": arch.value.decode()}

    def sync(self, stream=None) -> None:
        call("forge_sync", self.handle, stream)

    def streams_create(self, n: int):
        arr = (c_void_p * n)()
        call("forge_streams_create", self.handle, n, arr)
        return list(arr)

    def streams_fork(self, streams) -> None:
        arr = (c_void_p * len(streams))(*streams)
        call("forge_streams_fork", self.handle, len(streams), arr)

    def streams_join(self, streams) -> None:
        arr = (c_void_p * len(streams))(*streams)
        call("forge_streams_join", self.handle, len(streams), arr)

    def stream_wait(self, waiter, signaler) -> None:
        call("forge_stream_wait", self.handle, waiter, signaler)

    # -- events (device-side timing on a stream)
    def event(self):
        e = c_void_p()
        call("forge_event_create", self.handle, byref(e))
        return e

    def record(self, ev, stream=None) -> None:
        call("forge_event_record", self.handle, stream, ev)

    def elapsed_ms(self, start, end) -> float:
        ms = ctypes.c_float()
        call("forge_event_elapsed_ms", self.handle, start, end, byref(ms))
        return ms.value

    def event_destroy(self, ev) -> None:
        call("forge_event_destroy", self.handle, ev)

    # -- memory
    def empty(self, shape) -> DeviceArray:
        n = 1
        for s in shape:
            n *= int(s)
        sl = Slice()
        call("forge_alloc", self.handle, n, byref(sl))
        return DeviceArray(self, sl, shape)

    def zeros(self, shape) -> DeviceArray:
        n = 1
        for s in shape:
            n *= int(s)
        sl = Slice()
        call("forge_alloc_zeroed", self.handle, n, byref(sl))
        return DeviceArray(self, sl, shape)

    def array(self, host: np.ndarray) -> DeviceArray:
        host = np.ascontiguousarray(host, dtype=np.float32)
        return self.empty(host.shape).upload(host)

    def reserve(self, n: int, count: int) -> None:
        call("forge_reserve", self.handle, n, count)

    def pool_count(self, n: int) -> int:
        c = c_size_t()
        call("forge_pool_count", self.handle, n, byref(c))
        return c.value

    def free(self, a: DeviceArray) -> None:
        call("forge_free", self.handle, a.slice)
        a.slice = Slice(None, 0)

    def copy(self, dst: DeviceArray, src: DeviceArray, n: int | None = None, stream=None):
        call("forge_memcpy_d2d", self.handle, stream, dst.slice, src.slice,
             src.size if n is None else n)

    def fill(self, x: DeviceArray, value: float, stream=None) -> None:
        call("forge_fill", self.handle, stream, x.slice, value)

    # -- kernels (thin; shapes come from the DeviceArrays unless given)
    def gemm(self, A, B, C, M, N, K, stream=None) -> None:
        call("forge_gemm_f32", self.handle, stream, A.slice, B.slice, C.slice, M, N, K)

    def gemm_ex(self, A, B, C, M, N, K, trans_a=False, trans_b=False, stream=None,
                **epilogue) -> None:
        """forge_gemm_ex_f32; epilogue keywords as _epilogue (alpha, bias,
        residual, aux_mul, pre_out, activation, update, update_scale,
        aux_activation, row_parts_in, row_parts, row_n, row_eps, row_div,
        row_sumsq_out, col_sums_out, col_sums_param, col_sums_lr, row_sub)."""
        ep = _epilogue(**epilogue)
        call("forge_gemm_ex_f32", self.handle, stream, int(trans_a), int(trans_b), A.slice,
             B.slice, C.slice, M, N, K, byref(ep))

    def gemm_sum(self, As, Bs, C, M, N, K, trans_a=False, trans_b=False, stream=None,
                 **epilogue) -> None:
        """forge_gemm_sum_f32: C = epilogue(sum_z op(As[z]) op(Bs[z]))."""
        n = len(As)
        arr_a = (_lib.Slice * max(1, n))(*[a.slice for a in As])
        arr_b = (_lib.Slice * max(1, n))(*[b.slice for b in Bs])
        ep = _epilogue(**epilogue)
        call("forge_gemm_sum_f32", self.handle, stream, int(trans_a), int(trans_b), n, arr_a,
             arr_b, C.slice, M, N, K, byref(ep))

    def gemm_batch(self, problems, M, N, K, trans_a=False, trans_b=False, stream=None) -> None:
        """problems: [(A, B, C, dict of gemm_ex epilogue keywords), ...]."""
        arr = (_lib.GemmProblem * max(1, len(problems)))()
        for z, (A, B, C, ep) in enumerate(problems):
            arr[z] = _lib.GemmProblem(A.slice, B.slice, C.slice, _epilogue(**ep))
        call("forge_gemm_batch_f32", self.handle, stream, int(trans_a), int(trans_b), M, N, K,
             len(problems), arr)

    def gemm_tile(self, tile, A, B, C, M, N, K, stream=None) -> None:
        """forge_gemm_f32 through one named plain tile instance (tuning)."""
        call("forge_gemm_f32_tile", self.handle, stream, tile.encode(), A.slice, B.slice,
             C.slice, M, N, K)

    def gemm_kernel_name(self, M, N, K, trans_a=False, trans_b=False, fused=False) -> str:
        """Kernel gemm (fused=False) or gemm_ex (fused=True) launches for this
        shape with aligned operands ("<kernel>/split<N>" when split in K)."""
        buf = ctypes.create_string_buffer(128)
        call("forge_gemm_kernel_name", self.handle, int(trans_a), int(trans_b), M, N, K,
             int(fused), buf, len(buf))
        return buf.value.decode()

    def gemm_ex_tile(self, tile, A, B, C, M, N, K, trans_a=False, trans_b=False, stream=None,
                     **epilogue) -> None:
        """forge_gemm_ex_f32 through one named tile instance (testing)."""
        ep = _epilogue(**epilogue)
        call("forge_gemm_ex_f32_tile", self.handle, stream, tile.encode(), int(trans_a),
             int(trans_b), A.slice, B.slice, C.slice, M, N, K, byref(ep))

    def gemm_split(self, tile, splits, A, B, C, M, N, K, stream=None) -> None:
        call("forge_gemm_f32_split", self.handle, stream, tile.encode(), splits, A.slice,
             B.slice, C.slice, M, N, K)

    def transpose(self, x, out, rows, cols, stream=None) -> None:
        call("forge_transpose_f32", self.handle, stream, x.slice, out.slice, rows, cols)

    def softmax_rows(self, x, rows, cols, stream=None) -> None:
        call("forge_softmax_rows", self.handle, stream, x.slice, rows, cols)

    def softmax_rows_bwd(self, p, g, dx, rows, cols, stream=None) -> None:
        call("forge_softmax_rows_bwd", self.handle, stream, p.slice, g.slice, dx.slice, rows,
             cols)

    def layer_norm(self, x, rows, cols, gamma=None, beta=None, eps=1e-5, stream=None) -> None:
        call("forge_layer_norm_rows", self.handle, stream, x.slice, _sl(gamma), _sl(beta), rows,
             cols, eps)

    def layer_norm_out(self, x, y, rows, cols, gamma=None, beta=None, eps=1e-5,
                       stream=None) -> None:
        call("forge_layer_norm_rows_out", self.handle, stream, x.slice, y.slice, _sl(gamma),
             _sl(beta), rows, cols, eps)

    def layer_norm_bwd(self, x, dy, dx, rows, cols, gamma=None, dgamma=None, dbeta=None,
                       eps=1e-5, stream=None) -> None:
        call("forge_layer_norm_bwd", self.handle, stream, x.slice, dy.slice, _sl(gamma),
             dx.slice, _sl(dgamma), _sl(dbeta), rows, cols, eps)

    def layer_norm_bwd_sgd(self, x, dy, dx, rows, cols, lr, gamma=None, beta=None, dgamma=None,
                           dbeta=None, eps=1e-5, stream=None) -> None:
        call("forge_layer_norm_bwd_sgd", self.handle, stream, x.slice, dy.slice, _sl(gamma),
             _sl(beta), dx.slice, _sl(dgamma), _sl(dbeta), rows, cols, eps, lr)

    def rms_norm_bwd_sgd(self, x, dy, dx, rows, cols, lr, gamma=None, dgamma=None, eps=1e-5,
                         stream=None) -> None:
        call("forge_rms_norm_bwd_sgd", self.handle, stream, x.slice, dy.slice, _sl(gamma),
             dx.slice, _sl(dgamma), rows, cols, eps, lr)

    def layer_norm_bwd_sgd_dot(self, x, dy, dx, sub, dot, rows, cols, lr, dot_scale=1.0,
                               gamma=None, beta=None, dgamma=None, dbeta=None, eps=1e-5,
                               stream=None) -> None:
        """layer_norm_bwd_sgd plus dot[r] = dot_scale * sum_c dx[r,c] (x[r,c] - sub[r,c])."""
        call("forge_layer_norm_bwd_sgd_dot", self.handle, stream, x.slice, dy.slice, _sl(gamma),
             _sl(beta), dx.slice, _sl(dgamma), _sl(dbeta), _sl(sub), _sl(dot), rows, cols, eps,
             lr, dot_scale)

    def rms_norm_bwd_sgd_dot(self, x, dy, dx, sub, dot, rows, cols, lr, dot_scale=1.0,
                             gamma=None, dgamma=None, eps=1e-5, stream=None) -> None:
        """rms_norm_bwd_sgd plus the row dot of layer_norm_bwd_sgd_dot."""
        call("forge_rms_norm_bwd_sgd_dot", self.handle, stream, x.slice, dy.slice, _sl(gamma),
             dx.slice, _sl(dgamma), _sl(sub), _sl(dot), rows, cols, eps, lr, dot_scale)

    def sum_cols_sgd(self, m, rows, cols, lr, out=None, param=None, stream=None) -> None:
        call("forge_sum_cols_sgd", self.handle, stream, m.slice, rows, cols, _sl(out), _sl(param),
             lr)

    def rms_norm(self, x, rows, cols, gamma=None, eps=1e-5, stream=None) -> None:
        call("forge_rms_norm_rows", self.handle, stream, x.slice, _sl(gamma), rows, cols, eps)

    def rms_norm_out(self, x, y, rows, cols, gamma=None, eps=1e-5, stream=None) -> None:
        call("forge_rms_norm_rows_out", self.handle, stream, x.slice, y.slice, _sl(gamma), rows,
             cols, eps)

    def rms_norm_bwd(self, x, dy, dx, rows, cols, gamma=None, dgamma=None, eps=1e-5,
                     stream=None) -> None:
        call("forge_rms_norm_bwd", self.handle, stream, x.slice, dy.slice, _sl(gamma), dx.slice,
             _sl(dgamma), rows, cols, eps)

    def binary(self, l, r, o, op, n=None, stream=None) -> None:
        call("forge_binary", self.handle, stream, l.slice, r.slice, o.slice,
             o.size if n is None else n, op)

    def binary_assign(self, t, r, op, n=None, stream=None) -> None:
        call("forge_binary_assign", self.handle, stream, t.slice, r.slice,
             t.size if n is None else n, op)

    def binary_assign_by_rows(self, m, row, rows, cols, op, stream=None) -> None:
        call("forge_binary_assign_by_rows", self.handle, stream, m.slice, row.slice, rows, cols,
             op)

    def map(self, x, op, p0=0.0, n=None, stream=None) -> None:
        call("forge_map", self.handle, stream, x.slice, x.size if n is None else n, op, p0)

    def sum_rows(self, m, out, rows, cols, stream=None) -> None:
        call("forge_sum_rows", self.handle, stream, m.slice, out.slice, rows, cols)

    def sum_cols(self, m, out, rows, cols, stream=None) -> None:
        call("forge_sum_cols", self.handle, stream, m.slice, out.slice, rows, cols)

    def reduce_sum(self, x, out, n=None, stream=None) -> None:
        call("forge_reduce_sum", self.handle, stream, x.slice, x.size if n is None else n,
             out.slice)

    def map_sum(self, x, out, op, p0=0.0, n=None, stream=None) -> None:
        call("forge_map_sum", self.handle, stream, x.slice, x.size if n is None else n, op, p0,
             out.slice)

    def reduce_max(self, x, out, n=None, stream=None) -> None:
        call("forge_reduce_max", self.handle, stream, x.slice, x.size if n is None else n,
             out.slice)

    def fill_seq(self, x, ascending=True, n=None, stream=None) -> None:
        call("forge_fill_seq", self.handle, stream, x.slice, x.size if n is None else n,
             1 if ascending else 0)

    def causal_mask(self, m, rows, cols, stream=None) -> None:
        call("forge_causal_mask", self.handle, stream, m.slice, rows, cols)

    def softmax_rows_bwd_scaled(self, p, g, dx, rows, cols, scale, stream=None) -> None:
        call("forge_softmax_rows_bwd_scaled", self.handle, stream, p.slice, g.slice, dx.slice,
             rows, cols, scale)

    def activation_backward(self, dy, z, g, activation, n=None, stream=None) -> None:
        call("forge_activation_backward", self.handle, stream, dy.slice, z.slice, g.slice,
             g.size if n is None else n, activation)

    def sgd_update(self, param, grad, lr, n=None, stream=None) -> None:
        call("forge_sgd_update", self.handle, stream, param.slice, grad.slice,
             param.size if n is None else n, lr)

    def fill_random(self, x, seed, n=None, stream=None) -> None:
        call("forge_fill_random", self.handle, stream, x.slice, x.size if n is None else n, seed)

    def compare(self, l, r, out, n=None, stream=None) -> None:
        call("forge_compare", self.handle, stream, l.slice, r.slice, l.size if n is None else n,
             out.slice)
