"""The f32 arithmetic of the row kernels' LayerNorm and RMSNorm (forward
and backward), restated in numpy in the kernels' evaluation order: the
looping path (lane l sums columns l, l + 64, ... in turn) and the register
path (a lane sums its float4 groups, each as (x + y) + (z + w), and the
backward's products as fused multiply-adds), both reduced over the wave by
the same four DPP exchanges (quad [1,0,3,2], quad [2,3,0,1], half-row
mirror, row mirror) and a four-way combine of lanes 0, 16, 32 and 48.  On
the cases checked on the GPU it reproduces the kernels' largest errors
against the f64 oracle exactly; test_rowbounds.py uses it to show that the
tolerances of rowbounds.py cover f32 evaluation on ill-conditioned rows.
It is a model of the kernels for the tests, not a reference for them.
"""
import numpy as np

f = np.float32
_LANE = np.arange(64)
_DPP = [_LANE ^ 1, _LANE ^ 2, (_LANE & ~7) | (7 - (_LANE & 7)),
        (_LANE & ~15) | (15 - (_LANE & 15))]


def wave_sum(v):
    """Sum of v [rows, 64] over the lanes, as the kernels' wave_sum."""
    v = v.astype(f)
    for p in _DPP:
        v = (v + v[:, p]).astype(f)
    return ((v[:, 0] + v[:, 16]).astype(f) + (v[:, 32] + v[:, 48]).astype(f)).astype(f)


def _fma(a, b, c):
    # f32 * f32 is exact in f64; the f64 sum can round before the rounding to
    # f32 when the exponents differ by more than about 29 bits, where this
    # may differ from a fused multiply-add by one unit in the last place
    return (np.asarray(a, np.float64) * b + c).astype(f)


def _lanes_loop(t):
    rows, n = t.shape
    m = -(-n // 64)
    pad = np.zeros((rows, m * 64), f)
    pad[:, :n] = t
    s = np.zeros((rows, 64), f)
    for j in range(m):
        s = (s + pad[:, j * 64:(j + 1) * 64]).astype(f)
    return s


def _groups(t):
    rows, n = t.shape
    vpt = -(-n // 256)
    pad = np.zeros((rows, vpt * 256), f)
    pad[:, :n] = t
    return pad.reshape(rows, vpt, 64, 4)


def _sum4(g4):
    return ((g4[..., 0] + g4[..., 1]).astype(f) + (g4[..., 2] + g4[..., 3]).astype(f)).astype(f)


def _lanes(per):
    s = np.zeros(per.shape[:1] + (64,), f)
    for i in range(per.shape[1]):
        s = (s + per[:, i]).astype(f)
    return s


def _ungroup(g4, n):
    return g4.reshape(g4.shape[0], -1)[:, :n]


def layer_norm(x, dy, gamma, beta, eps=1e-5, register=False):
    """(forward y, backward dx) of LayerNorm rows, gamma/beta optional."""
    x = np.asarray(x, f)
    rows, n = x.shape
    nf = f(n)
    g_full = np.asarray(dy, f) if gamma is None else (np.asarray(dy, f) * gamma).astype(f)
    if register:
        X = _groups(x)
        ok = _groups(np.ones_like(x)) > 0
        mean = (wave_sum(_lanes(_sum4(X))) / nf).astype(f)[:, None, None, None]
        D = np.where(ok, (X - mean).astype(f), f(0))
        q = wave_sum(_lanes(_sum4((D * D).astype(f))))
    else:
        mean = (wave_sum(_lanes_loop(x)) / nf).astype(f)[:, None]
        D = (x - mean).astype(f)
        q = wave_sum(_lanes_loop((D * D).astype(f)))
    r = (f(1) / np.sqrt(((q / nf).astype(f) + f(eps)).astype(f)).astype(f)).astype(f)
    if register:
        XH = (D * r[:, None, None, None]).astype(f)
        y = XH
        if gamma is not None:
            y = (y * _groups(np.broadcast_to(gamma, x.shape).astype(f))).astype(f)
        if beta is not None:
            y = (y + _groups(np.broadcast_to(beta, x.shape).astype(f))).astype(f)
        G = _groups(g_full)
        sa = wave_sum(_lanes(_sum4(G)))
        per = (_fma(G[..., 0], XH[..., 0], (G[..., 1] * XH[..., 1]).astype(f))
               + _fma(G[..., 2], XH[..., 2], (G[..., 3] * XH[..., 3]).astype(f))).astype(f)
        sb = wave_sum(_lanes(per))
        scale = (r / nf).astype(f)[:, None, None, None]
        inner = _fma(nf, G, np.broadcast_to(-sa[:, None, None, None], G.shape))
        dx = (scale * _fma(XH, np.broadcast_to(-sb[:, None, None, None], G.shape), inner)).astype(f)
        return _ungroup(y, n), _ungroup(dx, n)
    XH = (D * r[:, None]).astype(f)
    y = XH
    if gamma is not None:
        y = (y * gamma).astype(f)
    if beta is not None:
        y = (y + beta).astype(f)
    sa = wave_sum(_lanes_loop(g_full))
    sb = wave_sum(_lanes_loop((g_full * XH).astype(f)))
    scale = (r / nf).astype(f)[:, None]
    t = ((nf * g_full).astype(f) - sa[:, None]).astype(f)
    dx = (scale * (t - (XH * sb[:, None]).astype(f)).astype(f)).astype(f)
    return y, dx


def rms_norm_backward(x, dy, gamma, eps=1e-5, register=False):
    """dx of RMSNorm rows, gamma optional."""
    x = np.asarray(x, f)
    rows, n = x.shape
    nf = f(n)
    g_full = np.asarray(dy, f) if gamma is None else (np.asarray(dy, f) * gamma).astype(f)
    if register:
        X, G = _groups(x), _groups(g_full)
        qq = (_fma(X[..., 0], X[..., 0], (X[..., 1] * X[..., 1]).astype(f))
              + _fma(X[..., 2], X[..., 2], (X[..., 3] * X[..., 3]).astype(f))).astype(f)
        dd = (_fma(X[..., 0], G[..., 0], (X[..., 1] * G[..., 1]).astype(f))
              + _fma(X[..., 2], G[..., 2], (X[..., 3] * G[..., 3]).astype(f))).astype(f)
        q, D = wave_sum(_lanes(qq)), wave_sum(_lanes(dd))
    else:
        q = wave_sum(_lanes_loop((x * x).astype(f)))
        D = wave_sum(_lanes_loop((x * g_full).astype(f)))
    rms = np.sqrt(((q / nf).astype(f) + f(eps)).astype(f)).astype(f)
    inv = (f(1) / rms).astype(f)
    c = ((((D / nf).astype(f) * inv).astype(f) * inv).astype(f) * inv).astype(f)
    gi = (g_full * inv[:, None]).astype(f)
    if register:
        return _fma(x, np.broadcast_to(-c[:, None], x.shape), gi)
    return (gi - (x * c[:, None]).astype(f)).astype(f)


def layer_norm_xhat(x, eps=1e-5, register=False):
    """The f32 xhat = (x - mean) * r of each row, as the kernels form it (the
    value their dgamma terms multiply)."""
    x = np.asarray(x, f)
    rows, n = x.shape
    nf = f(n)
    if register:
        X = _groups(x)
        ok = _groups(np.ones_like(x)) > 0
        mean = (wave_sum(_lanes(_sum4(X))) / nf).astype(f)[:, None, None, None]
        D = np.where(ok, (X - mean).astype(f), f(0))
        q = wave_sum(_lanes(_sum4((D * D).astype(f))))
    else:
        mean = (wave_sum(_lanes_loop(x)) / nf).astype(f)[:, None]
        D = (x - mean).astype(f)
        q = wave_sum(_lanes_loop((D * D).astype(f)))
    r = (f(1) / np.sqrt(((q / nf).astype(f) + f(eps)).astype(f)).astype(f)).astype(f)
    if register:
        return _ungroup((D * r[:, None, None, None]).astype(f), n)
    return (D * r[:, None]).astype(f)


def rms_norm_inv(x, eps=1e-5, register=False):
    """The f32 inv = 1 / sqrt(sum x^2 / n + eps) of each row, as the backward
    kernels form it."""
    x = np.asarray(x, f)
    n = x.shape[1]
    nf = f(n)
    if register:
        X = _groups(x)
        qq = (_fma(X[..., 0], X[..., 0], (X[..., 1] * X[..., 1]).astype(f))
              + _fma(X[..., 2], X[..., 2], (X[..., 3] * X[..., 3]).astype(f))).astype(f)
        q = wave_sum(_lanes(qq))
    else:
        q = wave_sum(_lanes_loop((x * x).astype(f)))
    rms = np.sqrt(((q / nf).astype(f) + f(eps)).astype(f)).astype(f)
    return (f(1) / rms).astype(f)
