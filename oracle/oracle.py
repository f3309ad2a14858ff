"""numpy front end of the CPU oracle (oracle/oxforge_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the timed
CPU baseline of bench.py.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product (oxide-forge_amd/) never
does.  See oxforge_oracle.h for the reference lines each function restates.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_size_t

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboxforge_oracle.so")

ADD, SUB, MUL, DIV = 0, 1, 2, 3
MAP_SCALE, MAP_ADD, MAP_GELU, MAP_GELU_D, MAP_RELU, MAP_RELU_D = 0, 1, 2, 3, 4, 5
MAP_SILU, MAP_SILU_D, MAP_EXP_SHIFT, MAP_HALF_SQ, MAP_IDENTITY = 6, 7, 8, 9, 10

_F = POINTER(c_float)
_D = POINTER(c_double)
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_set_threads": ([c_int], None),
            "orc_get_threads": ([], c_int),
            "orc_gemm": ([_F, _F, _F, c_size_t, c_size_t, c_size_t, c_int, c_int], None),
            "orc_gemm_f64": ([_F, _F, _D, c_size_t, c_size_t, c_size_t, c_int, c_int], None),
            "orc_transpose": ([_F, _F, c_size_t, c_size_t], None),
            "orc_softmax_rows": ([_F, c_size_t, c_size_t], None),
            "orc_softmax_rows_backward": ([_F, _F, _F, c_size_t, c_size_t], None),
            "orc_layer_norm_rows": ([_F, _F, _F, c_size_t, c_size_t, c_float], None),
            "orc_layer_norm_backward": ([_F, _F, _F, _F, _F, _F, c_size_t, c_size_t, c_float], None),
            "orc_rms_norm_rows": ([_F, _F, c_size_t, c_size_t, c_float], None),
            "orc_rms_norm_backward": ([_F, _F, _F, _F, _F, c_size_t, c_size_t, c_float], None),
            "orc_binary": ([_F, _F, _F, c_size_t, c_int], None),
            "orc_binary_assign": ([_F, _F, c_size_t, c_int], None),
            "orc_binary_assign_by_rows": ([_F, _F, c_size_t, c_size_t, c_int], None),
            "orc_map": ([_F, c_size_t, c_int, c_float], None),
            "orc_sum_rows": ([_F, _F, c_size_t, c_size_t], None),
            "orc_sum_cols": ([_F, _F, c_size_t, c_size_t], None),
            "orc_reduce_sum": ([_F, c_size_t], c_float),
            "orc_reduce_max": ([_F, c_size_t], c_float),
            "orc_fill_seq": ([_F, c_size_t, c_int], None),
            "orc_causal_mask": ([_F, c_size_t, c_size_t], None),
            "orc_activation_backward": ([_F, _F, _F, c_size_t, c_int], None),
            "orc_fill_random": ([_F, c_size_t, ctypes.c_uint32], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a: np.ndarray):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


# ------------------------------------------------------------- synthetic data
# ------------------------------------------------------------------- kernels
def gemm(A, B, trans_a=False, trans_b=False) -> np.ndarray:
    A, B = _f32(A), _f32(B)
    M = A.shape[1] if trans_a else A.shape[0]
    K = A.shape[0] if trans_a else A.shape[1]
    N = B.shape[0] if trans_b else B.shape[1]
    C = np.empty((M, N), dtype=np.float32)
    lib().orc_gemm(_p(A), _p(B), _p(C), M, N, K, int(trans_a), int(trans_b))
    return C


def gemm_f64(A, B, trans_a=False, trans_b=False) -> np.ndarray:
    A, B = _f32(A), _f32(B)
    M = A.shape[1] if trans_a else A.shape[0]
    K = A.shape[0] if trans_a else A.shape[1]
    N = B.shape[0] if trans_b else B.shape[1]
    C = np.empty((M, N), dtype=np.float64)
    lib().orc_gemm_f64(_p(A), _p(B), C.ctypes.data_as(_D), M, N, K, int(trans_a), int(trans_b))
    return C


def transpose(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty((x.shape[1], x.shape[0]), dtype=np.float32)
    lib().orc_transpose(_p(x), _p(out), x.shape[0], x.shape[1])
    return out


def softmax_rows(x) -> np.ndarray:
    y = _f32(x).copy()
    lib().orc_softmax_rows(_p(y), y.shape[0], y.shape[1])
    return y


def softmax_rows_backward(p, g) -> np.ndarray:
    p, g = _f32(p), _f32(g)
    dx = np.empty_like(p)
    lib().orc_softmax_rows_backward(_p(p), _p(g), _p(dx), p.shape[0], p.shape[1])
    return dx


def layer_norm(x, gamma=None, beta=None, eps=1e-5) -> np.ndarray:
    y = _f32(x).copy()
    g = None if gamma is None else _f32(gamma)
    b = None if beta is None else _f32(beta)
    lib().orc_layer_norm_rows(_p(y), _p(g), _p(b), y.shape[0], y.shape[1], eps)
    return y


def layer_norm_backward(x, dy, gamma=None, eps=1e-5, want_params=False):
    x, dy = _f32(x), _f32(dy)
    g = None if gamma is None else _f32(gamma)
    dx = np.empty_like(x)
    dg = np.empty(x.shape[1], np.float32) if want_params else None
    db = np.empty(x.shape[1], np.float32) if want_params else None
    lib().orc_layer_norm_backward(_p(x), _p(dy), _p(g), _p(dx), _p(dg), _p(db), x.shape[0],
                                  x.shape[1], eps)
    return (dx, dg, db) if want_params else dx


def rms_norm(x, gamma=None, eps=1e-5) -> np.ndarray:
    y = _f32(x).copy()
    g = None if gamma is None else _f32(gamma)
    lib().orc_rms_norm_rows(_p(y), _p(g), y.shape[0], y.shape[1], eps)
    return y


def rms_norm_backward(x, dy, gamma=None, eps=1e-5, want_params=False):
    x, dy = _f32(x), _f32(dy)
    g = None if gamma is None else _f32(gamma)
    dx = np.empty_like(x)
    dg = np.empty(x.shape[1], np.float32) if want_params else None
    lib().orc_rms_norm_backward(_p(x), _p(dy), _p(g), _p(dx), _p(dg), x.shape[0], x.shape[1],
                                eps)
    return (dx, dg) if want_params else dx


def binary(l, r, op) -> np.ndarray:
    l, r = _f32(l), _f32(r)
    o = np.empty_like(l)
    lib().orc_binary(_p(l), _p(r), _p(o), l.size, op)
    return o


def binary_assign(t, r, op) -> np.ndarray:
    t = _f32(t).copy()
    lib().orc_binary_assign(_p(t), _p(_f32(r)), t.size, op)
    return t


def binary_assign_by_rows(m, row, op) -> np.ndarray:
    m = _f32(m).copy()
    lib().orc_binary_assign_by_rows(_p(m), _p(_f32(row)), m.shape[0], m.shape[1], op)
    return m


def map_(x, op, p0=0.0) -> np.ndarray:
    y = _f32(x).copy()
    lib().orc_map(_p(y), y.size, op, p0)
    return y


def sum_rows(m) -> np.ndarray:
    m = _f32(m)
    out = np.empty(m.shape[0], np.float32)
    lib().orc_sum_rows(_p(m), _p(out), m.shape[0], m.shape[1])
    return out


def sum_cols(m) -> np.ndarray:
    m = _f32(m)
    out = np.empty(m.shape[1], np.float32)
    lib().orc_sum_cols(_p(m), _p(out), m.shape[0], m.shape[1])
    return out


def reduce_sum(x) -> float:
    x = _f32(x)
    return float(lib().orc_reduce_sum(_p(x), x.size))


def reduce_max(x) -> float:
    x = _f32(x)
    return float(lib().orc_reduce_max(_p(x), x.size))


def fill_seq(n, ascending=True) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_seq(_p(out), n, int(ascending))
    return out


def activation_backward(dy, z, derivative_op) -> np.ndarray:
    dy, z = _f32(dy), _f32(z)
    g = np.empty_like(dy)
    lib().orc_activation_backward(_p(dy), _p(z), _p(g), dy.size, derivative_op)
    return g


def fill_random(n, seed) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_random(_p(out), n, seed)
    return out


def causal_mask(m) -> np.ndarray:
    m = _f32(m).copy()
    lib().orc_causal_mask(_p(m), m.shape[0], m.shape[1])
    return m


# ------------------------------------------------------------ block forward
def transformer_forward(p, X, rms=True):
    """The single-head Post-Norm block forward as the reference launches it
    (inference.rs:76-108, attention.rs:258-281, 359-401, linear.rs:185-230):
    every step is one C kernel above, in f32 with f64-accumulated products.
    p maps slot names (WQ, BQ, WK, BK, WV, BV, POS, W1, B1, W2, B2, WO, BO) to
    arrays; biases may be None.  The multithreaded host mirror of the layer
    that bench.py times."""
    norm = rms_norm if rms else layer_norm

    def linear(x, w, b, act_op=None):
        z = gemm(x, w)
        if b is not None:
            z = binary_assign_by_rows(z, b, ADD)
        return map_(z, act_op) if act_op is not None else z

    xp = binary(X, p["POS"], ADD)
    q = linear(xp, p["WQ"], p.get("BQ"))
    k = linear(xp, p["WK"], p.get("BK"))
    v = linear(xp, p["WV"], p.get("BV"))
    s = map_(gemm(q, k, trans_b=True), MAP_SCALE, float(1.0 / np.sqrt(np.float32(q.shape[1]))))
    pmat = softmax_rows(s)
    h1 = norm(binary(xp, gemm(pmat, v), ADD))
    f = linear(linear(h1, p["W1"], p.get("B1"), MAP_GELU), p["W2"], p.get("B2"))
    h2 = norm(binary(h1, f, ADD))
    return linear(h2, p["WO"], p.get("BO"))


# ---------------------------------------------------------- training step
def transformer_training_step(p, X, dY, lr, rms=False):
    """One TrainingTransformer step as the reference launches it: forward
    (encoder.rs:114-131, attention.rs:258-281), backward (encoder.rs:133-186;
    the output and FFN layers through Linear::backward / input_gradient /
    learn, linear.rs:232-306, 350-444, with the FFN pre-activation recomputed
    as mlp.rs:136-139 does; attention.rs:283-321 and the Q/K/V projections of
    attention.rs:104-144) and every SGD step, each step one C kernel above in
    f32 with f64-accumulated products, transposes materialised where the
    reference materialises them.  Norms take the gamma/beta extension (G1,
    BE1, G2, BE2 in p, None for the reference's parameterless norm).

    Returns (output, dX, grads, new_params): grads keyed like p (each
    parameter's gradient before its update), new_params the parameters after
    the step.  The multithreaded host mirror of the C5 layer that bench.py
    times."""
    def norm_fwd(x, g, b):
        return rms_norm(x, g) if rms else layer_norm(x, g, b)

    def norm_bwd(x, dy, g):
        if rms:
            dx, dg = rms_norm_backward(x, dy, g, want_params=True)
            return dx, dg, None
        return layer_norm_backward(x, dy, g, want_params=True)

    def affine(x, w, b):
        z = gemm(x, w)
        return binary_assign_by_rows(z, b, ADD) if b is not None else z

    def sgd(param, grad):
        # clone, scale by lr, subtract (linear.rs:385-390, encoder.rs:180-184)
        return binary(param, map_(grad, MAP_SCALE, float(lr)), SUB)

    def bias_grad(g):
        # transpose, then sum_rows (linear.rs:267-272)
        return sum_rows(transpose(g))

    def input_gradient(g, w):
        return gemm(g, transpose(w))  # linear.rs:417-444

    def weight_gradient(x, g):
        return gemm(transpose(x), g)  # linear.rs:373-384

    grads, new = {}, dict(p)
    # forward
    xp = binary(X, p["POS"], ADD)
    q = affine(xp, p["WQ"], p.get("BQ"))
    k = affine(xp, p["WK"], p.get("BK"))
    v = affine(xp, p["WV"], p.get("BV"))
    scale = float(1.0 / np.sqrt(np.float32(q.shape[1])))
    pmat = softmax_rows(map_(gemm(q, transpose(k)), MAP_SCALE, scale))
    pre1 = binary(xp, gemm(pmat, v), ADD)
    out1 = norm_fwd(pre1, p.get("G1"), p.get("BE1"))
    h1 = map_(affine(out1, p["W1"], p.get("B1")), MAP_GELU)
    pre2 = binary(out1, affine(h1, p["W2"], p.get("B2")), ADD)
    enc = norm_fwd(pre2, p.get("G2"), p.get("BE2"))
    out = affine(enc, p["WO"], p.get("BO"))

    # output projection (identity activation)
    g_o = np.array(dY, np.float32, copy=True)
    if p.get("BO") is not None:
        grads["BO"] = bias_grad(g_o)
    d_enc = input_gradient(g_o, p["WO"])
    grads["WO"] = weight_gradient(enc, g_o)
    new["WO"] = sgd(p["WO"], grads["WO"])
    if p.get("BO") is not None:
        new["BO"] = sgd(p["BO"], grads["BO"])
    second, grads["G2"], grads["BE2"] = norm_bwd(pre2, d_enc, p.get("G2"))

    # FFN: layer 2 (identity), then layer 1 (GELU, pre-activation recomputed)
    g2 = second.copy()
    if p.get("B2") is not None:
        grads["B2"] = bias_grad(g2)
    dh1 = input_gradient(g2, p["W2"])
    grads["W2"] = weight_gradient(h1, g2)
    new["W2"] = sgd(p["W2"], grads["W2"])
    if p.get("B2") is not None:
        new["B2"] = sgd(p["B2"], grads["B2"])
    z1 = affine(out1, p["W1"], p.get("B1"))
    g1 = binary(dh1, map_(z1, MAP_GELU_D), MUL)
    if p.get("B1") is not None:
        grads["B1"] = bias_grad(g1)
    d_out1 = input_gradient(g1, p["W1"])
    grads["W1"] = weight_gradient(out1, g1)
    new["W1"] = sgd(p["W1"], grads["W1"])
    if p.get("B1") is not None:
        new["B1"] = sgd(p["B1"], grads["B1"])
    first = binary(second, d_out1, ADD)

    # attention
    r, grads["G1"], grads["BE1"] = norm_bwd(pre1, first, p.get("G1"))
    dp = gemm(r, transpose(v))
    dv = gemm(transpose(pmat), r)
    ds = map_(softmax_rows_backward(pmat, dp), MAP_SCALE, scale)
    dq = gemm(ds, k)
    dk = gemm(transpose(ds), q)
    proj = None
    for w, b, g in (("WQ", "BQ", dq), ("WK", "BK", dk), ("WV", "BV", dv)):
        if p.get(b) is not None:
            grads[b] = bias_grad(g)
        ig = input_gradient(g, p[w])
        proj = ig if proj is None else binary(proj, ig, ADD)
        grads[w] = weight_gradient(xp, g)
        new[w] = sgd(p[w], grads[w])
        if p.get(b) is not None:
            new[b] = sgd(p[b], grads[b])
    dxp = binary(r, proj, ADD)
    grads["POS"] = dxp
    new["POS"] = sgd(p["POS"], dxp)
    for n in ("G1", "BE1", "G2", "BE2"):
        if p.get(n) is None:
            grads[n] = None
        elif grads.get(n) is not None:
            new[n] = sgd(p[n], grads[n])
    return out, dxp, grads, new
