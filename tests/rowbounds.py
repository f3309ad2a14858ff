"""Rounding-error bounds of the f32 row-norm formulas (row.rs:115-177,
239-347, 349-468 as the row kernels evaluate them), used by the random-shape
tests as tolerances where they exceed the fixed bar.

A norm of a row whose values nearly coincide has a large r =
1/sqrt(var + eps) (up to 1/sqrt(eps) = 316), and the f32 rounding of the
row's mean is then amplified by r (forward) or r^2 (backward): the
LayerNorm backward of the two-column row [-0.2205, -0.2578] has r = 53,
and an f32 evaluation of the reference's formula lands 4.7e-5 from the f64
value.  No f32 implementation meets a fixed 1e-5 absolute bar on such rows;
the bar is meant for X ~ N(0,1) at 1024 columns, where these bounds stay
below it (test_rowbounds.py), so it is unchanged there.

The bounds propagate one rounding (unit roundoff u = 2^-24) per f32
operation of the kernels' evaluation order.  A row sum passes a term through
at most k = ceil(n/64) + 8 additions (ceil(n/64) in its lane, six DPP levels,
a four-way combine).  The mean's error, which r amplifies, is taken at its
worst case, k u sum|x| / n; the other sums, which enter unamplified, at the
probabilistic sqrt(k) u (independent rounding errors add like a random
walk).  Two errors are common to a whole row and are carried apart from the
per-element roundings: the mean's rounding, which moves every xhat by
shift = r * dm (the centred values sum to zero, so sum d^2 moves only by
n dm^2), and the relative error of r, which scales every xhat alike; the
shift's products are kept to second order, as they alone remain on a
constant row, where xhat and B vanish.  Inputs are f32 arrays [rows, n];
statistics are taken in f64.  tolerance() applies a factor of 2 over the
bound and never goes below the fixed bar.
"""
import numpy as np

U = 2.0 ** -24
SAFETY = 2.0


def _depth(n):
    """Additions a term passes through in a wave-per-row sum of n values."""
    return -(-n // 64) + 8


def _sum_err(k):
    """Relative rounding error of a sum of unamplified terms: sqrt(k) u."""
    return np.sqrt(k) * U


def _ln_stats(x, eps):
    x = np.asarray(x, np.float64)
    n = x.shape[1]
    k = _depth(n)
    mu = x.mean(axis=1, keepdims=True)
    d = x - mu
    v = (d * d).mean(axis=1, keepdims=True)
    r = 1.0 / np.sqrt(v + eps)
    xh = d * r
    # mean: the row sum (worst case), then / n
    dm = k * U * np.abs(x).sum(axis=1, keepdims=True) / n + U * np.abs(mu)
    # q = sum d^2: the subtraction and the square of each term, the sum
    dq = (3.0 * U + _sum_err(k)) * (d * d).sum(axis=1, keepdims=True) + n * dm * dm
    dv = dq / n + U * v
    # r = 1 / sqrt(v + eps): the add, the square root and the division
    rr = 0.5 * r * r * (dv + U * (v + eps)) + 2.0 * U
    # xhat = (x - m) * r: the subtraction and the product, per element
    dxh = 2.0 * U * np.abs(xh)
    return n, k, r, xh, rr, dxh, r * dm


def layer_norm_forward_bound(x, gamma=None, beta=None, eps=1e-5):
    """y = (x - mean) * r * gamma + beta."""
    n, _, _, xh, rr, dxh, shift = _ln_stats(x, eps)
    g = np.ones(n) if gamma is None else np.asarray(gamma, np.float64)
    b = np.zeros(n) if beta is None else np.asarray(beta, np.float64)
    ex = dxh + (np.abs(xh) + shift) * rr + shift
    return np.abs(g) * ex + U * np.abs(xh * g) + U * (np.abs(xh * g + b) + np.abs(g) * ex)


def layer_norm_backward_bound(x, dy, gamma=None, eps=1e-5):
    """dx = r/n * (n g - A - xhat B), g = dy * gamma, A = sum g,
    B = sum g xhat."""
    n, k, r, xh, rr, dxh, shift = _ln_stats(x, eps)
    dy = np.asarray(dy, np.float64)
    g = dy if gamma is None else dy * np.asarray(gamma, np.float64)
    dg = U * np.abs(g)
    A = g.sum(axis=1, keepdims=True)
    B = (g * xh).sum(axis=1, keepdims=True)
    dA = (_sum_err(k) + U) * np.abs(g).sum(axis=1, keepdims=True)
    # xhat's error: per element, the common relative error of r, the shift
    ex = dxh + (np.abs(xh) + shift) * rr + shift
    # B = sum g xhat: the common errors move it by about (B + shift A) dr/r
    # and shift * A
    dB = ((np.abs(g) * dxh + np.abs(xh) * dg).sum(axis=1, keepdims=True)
          + (np.abs(B) + shift * np.abs(A)) * rr + shift * np.abs(A) + shift * dA
          + (_sum_err(k) + U) * (np.abs(g * xh).sum(axis=1, keepdims=True)
                                 + shift * np.abs(g).sum(axis=1, keepdims=True)))
    T = n * g - A - xh * B
    # xhat * B with both perturbed, to second order
    dxB = np.abs(B) * ex + (np.abs(xh) + ex) * dB
    dT = (n * dg + dA + dxB + U * np.abs(n * g - A) + U * (np.abs(T) + dxB))
    dx = r / n * T
    return r / n * dT + (np.abs(T) + dT) / n * r * rr + 2.0 * U * np.abs(dx)


def rms_norm_backward_bound(x, dy, gamma=None, eps=1e-5):
    """dx = g * inv - x * (D / n * inv^3), inv = 1/sqrt(sum x^2 / n + eps),
    D = sum x g, g = dy * gamma."""
    x = np.asarray(x, np.float64)
    n = x.shape[1]
    k = _depth(n)
    dy = np.asarray(dy, np.float64)
    g = dy if gamma is None else dy * np.asarray(gamma, np.float64)
    dg = U * np.abs(g)
    q = (x * x).sum(axis=1, keepdims=True)
    dq = (_sum_err(k) + U) * q
    s2 = q / n + eps
    ds2 = dq / n + 2.0 * U * s2
    rms = np.sqrt(s2)
    inv = 1.0 / rms
    drms = 0.5 * ds2 / rms + U * rms
    dinv = inv * inv * drms + U * inv
    D = (x * g).sum(axis=1, keepdims=True)
    dD = (np.abs(x) * dg).sum(axis=1, keepdims=True) + (_sum_err(k) + U) * np.abs(x * g).sum(
        axis=1, keepdims=True)
    c = D / n * inv ** 3
    dc = dD / n * inv ** 3 + 3.0 * np.abs(D) / n * inv * inv * dinv + 4.0 * U * np.abs(c)
    dx = g * inv - x * c
    return (np.abs(x) * dc + np.abs(g) * dinv + inv * dg + U * np.abs(g * inv)
            + U * np.abs(dx))


def tolerance(bound, bar=1e-5):
    """Per-element tolerance: the fixed bar, or SAFETY times the bound where
    that is larger."""
    return np.maximum(bar, SAFETY * bound)
