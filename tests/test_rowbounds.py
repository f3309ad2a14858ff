"""CPU checks of the row-norm tolerances (rowbounds.py) that the random-shape
GPU tests apply where a fixed 1e-5 bar is below what f32 arithmetic can
reach:
- at the distribution the fixed bar is set for (X ~ N(0,1), 1024 columns)
  the tolerance is the fixed bar itself;
- the kernels' f32 evaluation (f32rows.py, their order of operations) stays
  inside it on ill-conditioned rows: near-constant and constant rows with
  means up to 30, on the looping and the register path;
- planted mistakes in the formulas exceed it by orders of magnitude, so it
  does not hide a wrong term.
"""
import numpy as np
import pytest

import f32rows
import rowbounds as rb
from oracle import oracle as orc
from oxforge import synth

BAR = 1e-5


def c2_like(rows=256, cols=1024):
    x = synth.normal((rows, cols), 1)
    dy = synth.normal((rows, cols), 2)
    gam = synth.normal((cols,), 3, 1.0, 0.1)
    bet = synth.normal((cols,), 4, 0.0, 0.1)
    return x, dy, gam, bet


def test_fixed_bar_unchanged_at_standard_normal_rows():
    x, dy, gam, bet = c2_like()
    for b in (rb.layer_norm_forward_bound(x, gam, bet), rb.layer_norm_backward_bound(x, dy, gam),
              rb.rms_norm_backward_bound(x, dy, gam)):
        assert np.all(rb.tolerance(b) == BAR)


def test_seed_case_reproduced():
    """The random-shape case that exceeded the fixed bar on the GPU: rows of
    two columns, one of them [-0.2205, -0.2578] (r = 53).  The f32 model
    gives the kernels' error, which the tolerance covers."""
    x = synth.normal((87, 2), 14403)
    dy = synth.normal((87, 2), 14453)
    gam = synth.normal((2,), 3, 1.0, 0.1)
    bet = synth.normal((2,), 4, 0.0, 0.1)
    _, dx = f32rows.layer_norm(x, dy, gam, bet)
    ref = orc.layer_norm_backward(x, dy, gam)
    err = np.abs(dx.astype(np.float64) - ref)
    assert err.max() == pytest.approx(4.696846008300781e-05, rel=1e-6)
    assert err.max() > BAR
    assert np.all(err <= rb.tolerance(rb.layer_norm_backward_bound(x, dy, gam)))


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8, 12, 33, 64, 256, 1024])
def test_f32_evaluation_within_tolerance_on_ill_conditioned_rows(n):
    rng = np.random.default_rng(100 + n)
    rows = 48 if n >= 256 else 120
    worst = 0.0
    for spread in (1.0, 1e-2, 1e-4, 1e-5, 0.0):
        m = rng.normal(0, 1, (rows, 1)) * rng.choice([1, 3, 10, 30], (rows, 1))
        x = (m + spread * rng.normal(0, 1, (rows, n))).astype(np.float32)
        dy = rng.normal(0, 1, (rows, n)).astype(np.float32)
        affine = spread != 1e-4
        gam = (1 + 0.1 * rng.normal(0, 1, n)).astype(np.float32) if affine else None
        bet = (0.1 * rng.normal(0, 1, n)).astype(np.float32) if affine else None
        for register in ((False, True) if n % 4 == 0 else (False,)):
            y, dx = f32rows.layer_norm(x, dy, gam, bet, register=register)
            dx2 = f32rows.rms_norm_backward(x, dy, gam, register=register)
            for got, ref, b in (
                    (y, orc.layer_norm(x, gam, bet), rb.layer_norm_forward_bound(x, gam, bet)),
                    (dx, orc.layer_norm_backward(x, dy, gam),
                     rb.layer_norm_backward_bound(x, dy, gam)),
                    (dx2, orc.rms_norm_backward(x, dy, gam),
                     rb.rms_norm_backward_bound(x, dy, gam))):
                err = np.abs(got.astype(np.float64) - ref)
                tol = rb.tolerance(b)
                assert np.all(err <= tol), (n, spread, register, float((err / tol).max()))
                worst = max(worst, float((err / tol).max()))
    print(f"n={n}: largest error / tolerance {worst:.3f}")


def _ln_parts(x, ddof=0, eps=1e-5):
    x = np.asarray(x, np.float64)
    d = x - x.mean(axis=1, keepdims=True)
    r = 1.0 / np.sqrt((d * d).sum(axis=1, keepdims=True) / (x.shape[1] - ddof) + eps)
    return d * r, r


def _planted(x, dy, gam, bet):
    """Each entry: (wrong result, oracle result, tolerance)."""
    n = x.shape[1]
    xh, r = _ln_parts(x)
    xh1, r1 = _ln_parts(x, ddof=1)
    g = np.asarray(dy, np.float64) * gam
    A = g.sum(axis=1, keepdims=True)
    B = (g * xh).sum(axis=1, keepdims=True)
    B1 = (g * xh1).sum(axis=1, keepdims=True)
    xx = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt((xx * xx).mean(axis=1, keepdims=True) + 1e-5)
    D = (xx * g).sum(axis=1, keepdims=True)
    tf = rb.tolerance(rb.layer_norm_forward_bound(x, gam, bet))
    tb = rb.tolerance(rb.layer_norm_backward_bound(x, dy, gam))
    tr = rb.tolerance(rb.rms_norm_backward_bound(x, dy, gam))
    rf, rbk, rr = (orc.layer_norm(x, gam, bet), orc.layer_norm_backward(x, dy, gam),
                   orc.rms_norm_backward(x, dy, gam))
    return {
        "forward, sample variance": (xh1 * gam + bet, rf, tf),
        "forward, beta dropped": (xh * gam, rf, tf),
        "backward, A dropped": (r / n * (n * g - xh * B), rbk, tb),
        "backward, sign of xhat B": (r / n * (n * g - A + xh * B), rbk, tb),
        "backward, sample variance": (r1 / n * (n * g - A - xh1 * B1), rbk, tb),
        "rms backward, inv^2": (g * inv - xx * D / n * inv ** 2, rr, tr),
        "rms backward, correction dropped": (g * inv, rr, tr),
    }


@pytest.mark.parametrize("cols", [2, 7, 1024, 3000])
def test_planted_mistakes_exceed_tolerance(cols):
    if cols == 1024:
        x, dy, gam, bet = c2_like(128, cols)
    else:
        x, dy = synth.normal((300, cols), 5), synth.normal((300, cols), 6)
        gam, bet = synth.normal((cols,), 3, 1.0, 0.1), synth.normal((cols,), 4, 0.0, 0.1)
    for name, (wrong, ref, tol) in _planted(x, dy, gam, bet).items():
        assert (np.abs(wrong - ref) / tol).max() > 50, name
