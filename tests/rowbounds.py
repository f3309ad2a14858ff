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


# ------------------------------------------------------------ column sums
# dgamma = sum over rows of dy * xhat (RMSNorm: dy * x * inv) and dbeta =
# sum of dy (the gamma/beta extension of row.rs:239-347, 398-468) are column
# sums of `rows` terms, taken by the norm backward kernels in a fixed tree:
#   1. each wave walks its rows grid-stride and accumulates every column in a
#      register chain (register path: a fused multiply-add per dgamma term;
#      looping path: the product, then the add);
#   2. the register path adds its workgroup's waves in LDS, wave 0 first;
#      the looping path keeps one partial row per wave;
#   3. a final pass sums the partial rows (a further chunked pass first when
#      there are more than 512 of them: the float4 first pass when the columns
#      and outputs allow it).
# The bound is the running error bound of that tree: every rounded addition
# contributes at most u |s| for its exact result s (a first-order bound,
# Higham, "Accuracy and Stability of Numerical Algorithms", 2nd ed., 4.2),
# plus each term's own error, which a sum passes on unchanged.  norm_bwd_plan
# restates the host's choice of grid (runtime.cpp row_launch, sum_cols_impl)
# so the tree is the one the kernels run.

def norm_bwd_plan(rows, cols, cu_count, layer, aligned=True):
    """Grid of the dgamma/dbeta partial pass: 'reg' (one partial row per
    workgroup of `waves` waves) or 'loop' (one per wave of four)."""
    vpt = 0
    if aligned and cols % 4 == 0 and cols > 0:
        for v in (1, 2, 4, 8, 16):
            if cols <= 256 * v:
                vpt = v
                break
    if vpt > 8:
        vpt = 0
    p4 = vpt == 4 and rows >= 256 * cu_count
    waves = (4 if p4 else 8) if vpt else 4
    per_cu = 2 if (p4 and layer) else 1
    grid = min(-(-rows // waves), max(64, cu_count) * per_cu)
    return {"kind": "reg" if vpt else "loop", "grid": grid, "waves": waves,
            "partial_rows": grid if vpt else grid * 4}


def _sum_cols_chunks(rows, cols, vec):
    if rows <= 512:
        return 1
    per_block = 256 if vec else 64
    gx = -(-cols // per_block)
    want = max(1, 8192 // max(1, gx))
    by_rows = -(-rows // 16)
    return max(2, min(want, by_rows, 512))


def _sum_cols_part_plan(rows, cols, loads=16, target=512):
    """Grid of the float4 first pass (runtime.cpp sum_cols_part_plan):
    (rows per chunk, chunks) for workgroups of 64 columns, 16 row slots and
    `loads` loads per slot per batch."""
    gx = -(-cols // 64)
    batch = 16 * loads
    batches = -(-rows // batch)
    chunks = min(max(1, target // gx), batches, 256)
    rpc = -(-batches // chunks) * batch
    return rpc, -(-rows // rpc)


def _uses_part(rows, cols, aligned):
    """forge_sum_cols' float4 first pass: more than 512 rows of float4
    columns, every operand 16-byte aligned (runtime.cpp sum_cols_impl)."""
    return aligned and cols % 4 == 0 and _sum_cols_chunks(rows, cols, True) > 1


def _halving(S, err):
    """Halving tree over the first axis (slot s + st into s for st = n/2,
    ..., 1): (sums, err plus every rounded partial sum)."""
    st = S.shape[0] // 2
    while st:
        S = S[:st] + S[st:2 * st]
        err = err + np.abs(S).sum(axis=0)
        st //= 2
    return S[0], err


def _sum_cols_part(T):
    """forge_sum_cols_p over T [rows, cols]: per chunk, 16 slot chains (rows
    s, s + 16, ...) and a halving tree; with several chunks the final pass
    over the partial rows.  Returns the sum of every rounded partial sum."""
    rows, cols = T.shape
    rpc, chunks = _sum_cols_part_plan(rows, cols)
    err = np.zeros(cols)
    parts = []
    for r0 in range(0, rows, rpc):
        S, e1 = _chains(T[r0:r0 + rpc], 16, False)
        v, err = _halving(S, err + e1)
        parts.append(v)
    if chunks == 1:
        return err
    _, e2 = _final_pass(np.array(parts), True)
    return err + e2


def _chains(T, n_chains, first_rounds):
    """Grid-stride chains: chain c sums rows c, c + n_chains, ... of T
    [rows, cols] in order.  Returns (the chains' exact sums [n_chains, cols],
    the sum over every rounded step of |partial sum|); the first step of a
    chain rounds only when first_rounds (a fused multiply-add from 0)."""
    rows, cols = T.shape
    a = -(-rows // n_chains)
    P = np.zeros((a * n_chains, cols))
    P[:rows] = T
    valid = np.zeros(a * n_chains, bool)
    valid[:rows] = True
    S = np.cumsum(P.reshape(a, n_chains, cols), axis=0)
    mask = valid.reshape(a, n_chains)
    if not first_rounds:
        mask = mask.copy()
        mask[0] = False
    err = (np.abs(S) * mask[:, :, None]).sum(axis=(0, 1))
    return S[-1], err


def _final_pass(Pm, vec):
    """sum_cols_final_v (64 slots of rows s, s + 64, ..., then a halving
    tree) or sum_cols_final (16 waves of rows w, w + 16, ..., then waves in
    order) over Pm [rows, cols]: (sums, sum of |partial sums|)."""
    slots = 64 if vec else 16
    S, err = _chains(Pm, slots, False)
    if vec:
        st = slots // 2
        while st:
            S = S[:st] + S[st:2 * st]
            err = err + np.abs(S).sum(axis=0)
            st //= 2
        return S[0], err
    C = np.cumsum(S, axis=0)
    return C[-1], err + np.abs(C[1:]).sum(axis=0)


def column_sum_bound(T, exact, plan, out_aligned=True, fma=False):
    """Bound on |computed - exact column sums| when the kernels sum the
    terms T [rows, cols] (f64 values of the f32 terms they form) in the tree
    of `plan`: |sum(T - exact)| (the terms' own error, exact) plus u times
    every rounded partial sum.  fma: each term is formed inside a fused
    multiply-add (register path), so a chain's first step rounds too.
    out_aligned: the outputs are 16-byte aligned (float4 final pass)."""
    T = np.asarray(T, np.float64)
    waves_total = plan["grid"] * plan["waves"]
    L1, err = _chains(T, waves_total, fma and plan["kind"] == "reg")
    if plan["kind"] == "reg":
        W = plan["waves"]
        C = np.cumsum(L1.reshape(plan["grid"], W, -1), axis=1)
        err = err + np.abs(C[:, 1:]).sum(axis=(0, 1))
        Pm = C[:, -1]
    else:
        Pm = L1
    # The partial rows sit in aligned scratch: the chunk pass is float4 when
    # cols % 4 == 0; the final pass and the one-launch form also need
    # aligned outputs.
    vec = T.shape[1] % 4 == 0
    prow = Pm.shape[0]
    if _uses_part(prow, T.shape[1], out_aligned):
        err = err + _sum_cols_part(Pm)
        return np.abs((T - np.asarray(exact, np.float64)).sum(axis=0)) + U * err
    chunks = _sum_cols_chunks(prow, T.shape[1], vec)
    if chunks > 1:
        rpc = -(-prow // chunks)
        chunks = -(-prow // rpc)
        parts = []
        for y in range(chunks):
            blk = Pm[y * rpc:(y + 1) * rpc]
            S, e1 = _chains(blk, 4, False)
            C = np.cumsum(S, axis=0)
            err = err + e1 + np.abs(C[1:]).sum(axis=0)
            parts.append(C[-1])
        Pm = np.array(parts)
    _, e2 = _final_pass(Pm, vec and out_aligned)
    return np.abs((T - np.asarray(exact, np.float64)).sum(axis=0)) + U * (err + e2)


def sum_cols_bound(m, aligned=True):
    """Bound on forge_sum_cols of m [rows, cols] (exact f32 inputs): the
    float4 first pass for more than 512 aligned float4 rows, otherwise the
    chunked first pass when rows > 512; then the final pass."""
    T = np.asarray(m, np.float64)
    rows, cols = T.shape
    if _uses_part(rows, cols, aligned):
        return U * _sum_cols_part(T)
    vec = aligned and cols % 4 == 0
    err = np.zeros(cols)
    Pm = T
    chunks = _sum_cols_chunks(rows, cols, vec)
    if chunks > 1:
        rpc = -(-rows // chunks)
        parts = []
        for r0 in range(0, rows, rpc):
            S, e1 = _chains(T[r0:r0 + rpc], 4, False)
            C = np.cumsum(S, axis=0)
            err = err + e1 + np.abs(C[1:]).sum(axis=0)
            parts.append(C[-1])
        Pm = np.array(parts)
    _, e2 = _final_pass(Pm, vec)
    return U * (err + e2)


def layer_norm_param_bounds(x, dy, cu_count, eps=1e-5, aligned=True, out_aligned=True):
    """Bounds on the kernels' dgamma = sum dy xhat and dbeta = sum dy: the
    terms use the kernels' own f32 xhat (f32rows.layer_norm_xhat), whose
    difference from the exact xhat enters exactly."""
    import f32rows

    x32 = np.asarray(x, np.float32)
    dy = np.asarray(dy, np.float32).astype(np.float64)
    rows, n = x32.shape
    plan = norm_bwd_plan(rows, n, cu_count, True, aligned)
    reg = plan["kind"] == "reg"
    xh = f32rows.layer_norm_xhat(x32, eps, register=reg).astype(np.float64)
    xd = x32.astype(np.float64)
    mu = xd.mean(axis=1, keepdims=True)
    exact_xh = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(axis=1, keepdims=True) + eps)
    t = dy * xh
    if not reg:
        t = t.astype(np.float32).astype(np.float64)  # the product rounds before the add
    bg = column_sum_bound(t, dy * exact_xh, plan, out_aligned, fma=True)
    bb = column_sum_bound(dy, dy, plan, out_aligned)
    return bg, bb


def rms_norm_param_bound(x, dy, cu_count, eps=1e-5, aligned=True, out_aligned=True):
    """Bound on the kernels' dgamma = sum dy (x inv), inv =
    1/sqrt(sum x^2 / n + eps) per row, with the kernels' f32 inv and x inv."""
    import f32rows

    x32 = np.asarray(x, np.float32)
    dy = np.asarray(dy, np.float32).astype(np.float64)
    rows, n = x32.shape
    plan = norm_bwd_plan(rows, n, cu_count, False, aligned)
    reg = plan["kind"] == "reg"
    inv = f32rows.rms_norm_inv(x32, eps, register=reg)
    xi = (x32 * inv[:, None]).astype(np.float32).astype(np.float64)
    xd = x32.astype(np.float64)
    exact = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + eps)
    t = dy * xi
    if not reg:
        t = t.astype(np.float32).astype(np.float64)
    return column_sum_bound(t, dy * exact, plan, out_aligned, fma=True)
