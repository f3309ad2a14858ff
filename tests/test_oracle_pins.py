"""Pins the CPU oracle (oracle/oxforge_oracle.c) before it is trusted.

The reference ships no tests, golden vectors or fixtures and cannot be built
here (it needs the un-vendored cuda-oxide git dependency and an NVIDIA GPU),
so each oracle function is pinned by what the mathematics fixes:
library routines (numpy f64 matmul, a textbook softmax/LayerNorm written in
f64 below), closed forms and invariants, exact small-integer cases, and
central finite differences for every backward.  Each check is chosen so a
plausible mistake (dropped term, wrong sign, transposed operand, wrong
normaliser) fails it.
"""
import numpy as np
import pytest

from oracle import oracle as orc

EPS = 1e-5


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ helpers
def softmax64(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def layer_norm64(x, g=None, b=None, eps=EPS):
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if g is not None:
        y = y * g
    if b is not None:
        y = y + b
    return y


def rms_norm64(x, g=None, eps=EPS):
    x = np.asarray(x, np.float64)
    y = x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return y * g if g is not None else y


def fd_grad(f, x, h=1e-6):
    """Central differences of the scalar f at x (f64)."""
    x = np.array(x, np.float64)
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp = x.copy()
        xm = x.copy()
        xp[i] += h
        xm[i] -= h
        g[i] = (f(xp) - f(xm)) / (2 * h)
    return g


def gelu64(x):
    s, c = np.float64(np.float32(0.7978846)), np.float64(np.float32(0.044715))
    return 0.5 * x * (1 + np.tanh(s * (x + c * x ** 3)))


# --------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (5, 7, 3), (33, 17, 65), (64, 48, 128)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_matches_numpy_f64(M, N, K, ta, tb):
    r = rng(M * 100 + N + K)
    A = r.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = r.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    assert np.allclose(orc.gemm_f64(A, B, ta, tb), ref, rtol=1e-12, atol=1e-12)
    assert np.array_equal(orc.gemm(A, B, ta, tb), ref.astype(np.float32))


def test_gemm_small_integers_exact_and_rank1():
    r = rng(1)
    A = r.integers(-16, 17, (40, 300)).astype(np.float32)
    B = r.integers(-16, 17, (300, 24)).astype(np.float32)
    exact = A.astype(np.int64) @ B.astype(np.int64)
    assert np.array_equal(orc.gemm(A, B), exact.astype(np.float32))
    u = r.uniform(-1, 1, (9, 1)).astype(np.float32)
    v = r.uniform(-1, 1, (1, 11)).astype(np.float32)
    assert np.array_equal(orc.gemm(u, v), (u.astype(np.float64) * v).astype(np.float32))


def test_gemm_not_transposed_by_mistake():
    # A non-symmetric, non-square product distinguishes A*B from B^T*A^T etc.
    A = np.arange(6, dtype=np.float32).reshape(2, 3)
    B = np.arange(12, dtype=np.float32).reshape(3, 4)
    assert np.array_equal(orc.gemm(A, B), np.array([[20, 23, 26, 29], [56, 68, 80, 92]], np.float32))


# ---------------------------------------------------------------- transpose
def test_transpose_index_map():
    x = np.arange(35, dtype=np.float32).reshape(5, 7)
    t = orc.transpose(x)
    assert t.shape == (7, 5)
    assert np.array_equal(t, x.T)
    assert np.array_equal(orc.transpose(t), x)


# ------------------------------------------------------------------ softmax
def test_softmax_library_and_invariants():
    r = rng(2)
    x = r.normal(0, 3, (7, 50)).astype(np.float32)
    y = orc.softmax_rows(x)
    assert np.allclose(y, softmax64(x), atol=1e-7, rtol=0)
    assert np.allclose(y.sum(axis=1), 1, atol=1e-6)
    assert np.allclose(orc.softmax_rows(x + np.float32(5)), y, atol=2e-7)  # shift invariance
    one_hot = np.full((1, 6), -1e4, np.float32)
    one_hot[0, 3] = 0
    assert np.array_equal(orc.softmax_rows(one_hot), np.eye(6, dtype=np.float32)[3:4])


def test_softmax_backward_finite_difference():
    r = rng(3)
    x = r.normal(0, 1, (3, 9))
    g = r.normal(0, 1, (3, 9))
    fd = fd_grad(lambda z: float((g * softmax64(z)).sum()), x)
    p = softmax64(x).astype(np.float32)
    dx = orc.softmax_rows_backward(p, g.astype(np.float32))
    assert np.allclose(dx, fd, atol=2e-6)
    # constant upstream gradient gives zero (rows of J sum to zero)
    assert np.allclose(orc.softmax_rows_backward(p, np.ones_like(p)), 0, atol=1e-7)


# ---------------------------------------------------------------- LayerNorm
def test_layer_norm_library_and_invariants():
    r = rng(4)
    x = r.normal(0, 2, (6, 40)).astype(np.float32)
    y = orc.layer_norm(x)
    assert np.allclose(y, layer_norm64(x), atol=1e-6)
    v = x.astype(np.float64).var(axis=1)
    assert np.allclose(y.astype(np.float64).sum(axis=1), 0, atol=1e-5)
    assert np.allclose((y.astype(np.float64) ** 2).mean(axis=1), v / (v + EPS), atol=1e-6)
    g = r.normal(1, 0.1, 40).astype(np.float32)
    b = r.normal(0, 0.1, 40).astype(np.float32)
    assert np.allclose(orc.layer_norm(x, g, b), layer_norm64(x, g, b), atol=1e-6)
    ones, zeros = np.ones(40, np.float32), np.zeros(40, np.float32)
    assert np.array_equal(orc.layer_norm(x, ones, zeros), y)  # affine reduces to reference


def test_layer_norm_backward_finite_difference():
    r = rng(5)
    x = r.normal(0, 1, (3, 8))
    dy = r.normal(0, 1, (3, 8))
    g = r.normal(1, 0.1, 8)
    b = r.normal(0, 0.1, 8)
    fdx = fd_grad(lambda z: float((dy * layer_norm64(z, g, b)).sum()), x)
    fdg = fd_grad(lambda gg: float((dy * layer_norm64(x, gg, b)).sum()), g)
    fdb = fd_grad(lambda bb: float((dy * layer_norm64(x, g, bb)).sum()), b)
    dx, dg, db = orc.layer_norm_backward(x.astype(np.float32), dy.astype(np.float32),
                                         g.astype(np.float32), want_params=True)
    assert np.allclose(dx, fdx, atol=5e-5)
    assert np.allclose(dg, fdg, atol=5e-5)
    assert np.allclose(db, fdb, atol=5e-5)
    # reference path (no gamma): dx is orthogonal to ones, and
    # sum(dx * xhat) = r * B * eps / (v + eps) with B = sum(dy * xhat).
    dx0 = orc.layer_norm_backward(x.astype(np.float32), dy.astype(np.float32)).astype(np.float64)
    xh = layer_norm64(x)
    v = x.var(axis=1)
    rstd = 1 / np.sqrt(v + EPS)
    B = (dy * xh).sum(axis=1)
    assert np.allclose(dx0.sum(axis=1), 0, atol=1e-5)
    assert np.allclose((dx0 * xh).sum(axis=1), rstd * B * EPS / (v + EPS), atol=1e-5)


# ------------------------------------------------------------------ RMSNorm
def test_rms_norm_library_and_invariants():
    r = rng(6)
    x = r.normal(0, 2, (5, 33)).astype(np.float32)
    y = orc.rms_norm(x)
    assert np.allclose(y, rms_norm64(x), atol=1e-6)
    ms = (x.astype(np.float64) ** 2).mean(axis=1)
    assert np.allclose((y.astype(np.float64) ** 2).mean(axis=1), ms / (ms + EPS), atol=1e-6)
    g = r.normal(1, 0.1, 33).astype(np.float32)
    assert np.allclose(orc.rms_norm(x, g), rms_norm64(x, g), atol=1e-6)


def test_rms_norm_backward_finite_difference():
    r = rng(7)
    x = r.normal(0, 1, (3, 7))
    dy = r.normal(0, 1, (3, 7))
    g = r.normal(1, 0.1, 7)
    fdx = fd_grad(lambda z: float((dy * rms_norm64(z, g)).sum()), x)
    fdg = fd_grad(lambda gg: float((dy * rms_norm64(x, gg)).sum()), g)
    dx, dg = orc.rms_norm_backward(x.astype(np.float32), dy.astype(np.float32),
                                   g.astype(np.float32), want_params=True)
    assert np.allclose(dx, fdx, atol=5e-5)
    assert np.allclose(dg, fdg, atol=5e-5)
    fd0 = fd_grad(lambda z: float((dy * rms_norm64(z)).sum()), x)
    assert np.allclose(orc.rms_norm_backward(x.astype(np.float32), dy.astype(np.float32)), fd0,
                       atol=5e-5)


# -------------------------------------------------------------- elementwise
@pytest.mark.parametrize("op,fn", [(orc.ADD, np.add), (orc.SUB, np.subtract),
                                   (orc.MUL, np.multiply), (orc.DIV, np.divide)])
def test_binary_ops_bit_exact(op, fn):
    r = rng(op)
    a = r.normal(0, 1, 1000).astype(np.float32)
    b = r.normal(0, 1, 1000).astype(np.float32)
    assert np.array_equal(orc.binary(a, b, op), fn(a, b))  # numpy f32: one rounding
    assert np.array_equal(orc.binary_assign(a, b, op), fn(a, b))
    m = a.reshape(40, 25)
    row = b[:25]
    assert np.array_equal(orc.binary_assign_by_rows(m, row, op), fn(m, row[None, :]))


def test_maps():
    r = rng(8)
    x = r.normal(0, 2, 2000).astype(np.float32)
    assert np.array_equal(orc.map_(x, orc.MAP_SCALE, 0.37), x * np.float32(0.37))
    assert np.array_equal(orc.map_(x, orc.MAP_ADD, -1.5), x + np.float32(-1.5))
    assert np.array_equal(orc.map_(x, orc.MAP_HALF_SQ), np.float32(0.5) * x * x)
    assert np.array_equal(orc.map_(x, orc.MAP_RELU), np.where(x > 0, x, 0).astype(np.float32))
    assert np.array_equal(orc.map_(x, orc.MAP_RELU_D), (x > 0).astype(np.float32))
    assert np.array_equal(orc.map_(x, orc.MAP_IDENTITY), x)
    xd = x.astype(np.float64)
    assert np.allclose(orc.map_(x, orc.MAP_GELU), gelu64(xd), rtol=1e-7, atol=1e-7)
    # derivatives against central differences of the forward formulas
    h = 1e-6
    fd_gelu = (gelu64(xd + h) - gelu64(xd - h)) / (2 * h)
    assert np.allclose(orc.map_(x, orc.MAP_GELU_D), fd_gelu, atol=1e-6)
    silu64 = lambda z: z / (1 + np.exp(-z))
    assert np.allclose(orc.map_(x, orc.MAP_SILU), silu64(xd), rtol=1e-7, atol=1e-7)
    fd_silu = (silu64(xd + h) - silu64(xd - h)) / (2 * h)
    assert np.allclose(orc.map_(x, orc.MAP_SILU_D), fd_silu, atol=1e-6)
    assert np.allclose(orc.map_(x, orc.MAP_EXP_SHIFT, 1.25), np.exp(xd - 1.25), rtol=1e-7)


# --------------------------------------------------------------- reductions
def test_reductions_exact_on_integers():
    r = rng(9)
    m = r.integers(-100, 101, (37, 53)).astype(np.float32)
    assert np.array_equal(orc.sum_rows(m), m.astype(np.int64).sum(axis=1).astype(np.float32))
    assert np.array_equal(orc.sum_cols(m), m.astype(np.int64).sum(axis=0).astype(np.float32))
    assert orc.reduce_sum(m) == float(m.astype(np.int64).sum())
    assert orc.reduce_max(m) == float(m.max())
    assert orc.reduce_sum(np.zeros(0, np.float32)) == 0.0
    assert orc.reduce_max(np.zeros(0, np.float32)) == float(np.finfo(np.float32).min)


def test_fills_and_mask():
    assert np.array_equal(orc.fill_seq(5, True), np.array([0, 1, 2, 3, 4], np.float32))
    assert np.array_equal(orc.fill_seq(5, False), np.array([5, 4, 3, 2, 1], np.float32))
    m = orc.causal_mask(np.zeros((4, 6), np.float32))
    ref = np.where(np.arange(6)[None, :] > np.arange(4)[:, None], -np.inf, 0).astype(np.float32)
    assert np.array_equal(m, ref)


def test_fill_random_hash_restated_independently():
    # common.rs:3-9 in wrapping u32 arithmetic, restated with numpy uint64
    # masks; elementwise.rs:40-41 divides by u32::MAX as f32.
    seed = 0xC0FFEE
    i = np.arange(5000, dtype=np.uint64)
    x = (seed + i) & 0xFFFFFFFF
    x = (x + (x << 13)) & 0xFFFFFFFF
    x = (x - (x >> 17)) & 0xFFFFFFFF
    x = (x * ((x << 5) & 0xFFFFFFFF)) & 0xFFFFFFFF
    ref = x.astype(np.float32) / np.float32(4294967295.0)
    assert np.array_equal(orc.fill_random(5000, seed), ref)


def test_fill_random_hash_known_answers():
    # Hand-derived values of common.rs:3-9 (wrapping u32):
    #   x=1: 1 + (1<<13) = 0x2001; 0x2001>>17 = 0; 0x2001 * (0x2001<<5) =
    #        8193 * 262176 = 2148007968 (< 2^32).
    #   x=2: 0x4002; >>17 = 0; 16386 * 524352 = 8592031872 = 2*2^32 + 2097280.
    #   x=0xFFFFFFFF: + (x<<13 = 0xFFFFE000) wraps to 0xFFFFDFFF; minus
    #        (0xFFFFDFFF>>17 = 0x7FFF) = 0xFFFF6000 = -40960; x<<5 = 0xFFEC0000
    #        = -1310720; product 53687091200 = 12*2^32 + 0x80000000.
    # elementwise.rs:40-41 hashes seed + index (wrapping) and divides by
    # u32::MAX as f32 (= 2^32), so 0x80000000 maps to exactly 0.5.
    two32 = np.float32(4294967295.0)
    got = orc.fill_random(3, 0)
    assert got[0] == 0.0
    assert got[1] == np.float32(2148007968) / two32
    assert got[2] == np.float32(2097280) / two32
    wrap = orc.fill_random(2, 0xFFFFFFFF)
    assert wrap[0] == np.float32(0.5)
    assert wrap[1] == 0.0  # seed + 1 wraps to 0


def test_activation_backward_is_dy_times_derivative():
    r = rng(11)
    dy = r.normal(0, 1, 500).astype(np.float32)
    z = r.normal(0, 2, 500).astype(np.float32)
    for op in (orc.MAP_GELU_D, orc.MAP_RELU_D, orc.MAP_SILU_D):
        assert np.array_equal(orc.activation_backward(dy, z, op), dy * orc.map_(z, op))
