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


def _slots_f32(blk, n=16):
    """n slot chains (rows s, s + n, ...) in f32, then the halving tree."""
    f = np.float32
    s = np.zeros((n, blk.shape[1]), f)
    for r in range(blk.shape[0]):
        s[r % n] = (s[r % n] + blk[r]).astype(f)
    st = n // 2
    while st:
        s = (s[:st] + s[st:2 * st]).astype(f)
        st //= 2
    return s[0]


def _sum_cols_part_f32(acc):
    """forge_sum_cols_p in f32: per chunk the slot chains and tree, then the
    float4 final pass (64 slots and the halving tree) over the partial rows."""
    rows, cols = acc.shape
    rpc, chunks = rb._sum_cols_part_plan(rows, cols)
    parts = np.array([_slots_f32(acc[r0:r0 + rpc]) for r0 in range(0, rows, rpc)])
    return parts[0] if chunks == 1 else _slots_f32(parts, 64)


def _tree_f32(T, plan, fma, out_aligned=True):
    """The kernels' column-sum tree evaluated in f32 (the order of
    rowbounds.column_sum_bound): wave chains (each step one rounding: a
    fused multiply-add on the register path), the workgroup's waves in
    order, the final pass's 64 slots and halving tree (or 16 waves in
    order)."""
    f = np.float32
    T = np.asarray(T, np.float64)
    rows, cols = T.shape
    nw = plan["grid"] * plan["waves"]
    a = -(-rows // nw)
    pad = np.zeros((a * nw, cols))
    pad[:rows] = T
    pad = pad.reshape(a, nw, cols)
    acc = np.zeros((nw, cols), f)
    for k in range(a):
        live = np.arange(nw) + k * nw < rows
        new = (acc.astype(np.float64) + pad[k]).astype(f)  # one rounding per step
        acc = np.where(live[:, None], new, acc)
    if plan["kind"] == "reg":
        acc = acc.reshape(plan["grid"], plan["waves"], cols)
        t = acc[:, 0]
        for w in range(1, plan["waves"]):
            t = (t + acc[:, w]).astype(f)
        acc = t
    prow = acc.shape[0]
    if rb._uses_part(prow, cols, out_aligned):
        return _sum_cols_part_f32(acc)
    chunks = rb._sum_cols_chunks(prow, cols, cols % 4 == 0)
    if chunks > 1:
        # first pass: chunks of rpc rows, four waves of rows r0 + w, r0 + w + 4,
        # ..., then the waves in order
        rpc = -(-prow // chunks)
        parts = []
        for r0 in range(0, prow, rpc):
            blk = acc[r0:r0 + rpc]
            w4 = np.zeros((4, cols), f)
            for r in range(blk.shape[0]):
                w4[r % 4] = (w4[r % 4] + blk[r]).astype(f)
            t = w4[0]
            for w in range(1, 4):
                t = (t + w4[w]).astype(f)
            parts.append(t)
        acc = np.array(parts)
    vec = cols % 4 == 0 and out_aligned
    slots = 64 if vec else 16
    s = np.zeros((slots, cols), f)
    for r in range(acc.shape[0]):
        s[r % slots] = (s[r % slots] + acc[r]).astype(f)
    if vec:
        st = slots // 2
        while st:
            s = (s[:st] + s[st:2 * st]).astype(f)
            st //= 2
        return s[0]
    t = s[0]
    for w in range(1, slots):
        t = (t + s[w]).astype(f)
    return t


@pytest.mark.parametrize("rows,cols,aligned", [(4096, 256, True), (600, 1001, False),
                                               (70, 64, True), (3000, 2560, True)])
def test_column_sum_bound_covers_f32_tree_and_catches_a_dropped_row(rows, cols, aligned):
    """dgamma / dbeta bounds (rowbounds.layer_norm_param_bounds): the f32
    evaluation of the kernels' summation tree over the kernels' own f32 xhat
    lands inside the bound on every column, and a planted mistake (the last
    row's terms left out) exceeds twice the bound."""
    import f32rows

    x = synth.normal((rows, cols), 5)
    dy = synth.normal((rows, cols), 6)
    cu = 256
    bg, bb = rb.layer_norm_param_bounds(x, dy, cu, aligned=aligned)
    plan = rb.norm_bwd_plan(rows, cols, cu, True, aligned)
    reg = plan["kind"] == "reg"
    xh = f32rows.layer_norm_xhat(x, register=reg).astype(np.float64)
    t = dy.astype(np.float64) * xh
    if not reg:
        t = t.astype(np.float32).astype(np.float64)
    _, rdg, rdb = orc.layer_norm_backward(x, dy, None, want_params=True)
    got_g = _tree_f32(t, plan, True).astype(np.float64)
    got_b = _tree_f32(dy, plan, False).astype(np.float64)
    assert np.all(np.abs(got_g - rdg) <= bg)
    assert np.all(np.abs(got_b - rdb) <= bb)
    # the bound is a rounding bound, not a slack: a missing row is far outside
    t2 = t.copy()
    t2[-1] = 0.0
    bad = _tree_f32(t2, plan, True).astype(np.float64)
    assert np.any(np.abs(bad - rdg) > rb.SAFETY * bg)
