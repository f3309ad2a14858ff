"""The attention backward's softmax step as the training step computes it,
against the reference's order, in f64 (no GPU).

The reference (attention.rs:283-321 with row.rs:216-236) forms dP = R V^T,
then dS = P * (dP - D) * s with D_r = sum_j P_rj dP_rj over each [Sk] row.
The training step instead takes D_r = sum_c R_rc (pre_norm - X)_rc from the
[S, H] operands its norm backward already streams (pre_norm = P V + X, the
forward's A.V product with the input X as residual) and forms
dS = P * (s dP - s D) in the dP product's epilogue.  The two agree in exact
arithmetic; this pins that identity (and that the operands are the ones the
library passes) so that a plausible slip -- the residual not subtracted, the
sum taken over the wrong axis or not at all -- fails.
"""
import numpy as np


def softmax64(x):
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def reference_ds(P, R, V, s):
    dP = R @ V.T
    D = (P * dP).sum(axis=1, keepdims=True)
    return (P * (dP - D)) * s


def folded_ds(P, R, V, X, s):
    pre = P @ V + X
    D = (R * (pre - X)).sum(axis=1, keepdims=True)
    dP = R @ V.T
    return P * (s * dP - s * D)


def test_folded_softmax_backward_equals_reference_order():
    rng = np.random.default_rng(5)
    for S, Sk, H in ((48, 40, 24), (64, 64, 64), (7, 130, 9)):
        P = softmax64(rng.normal(size=(S, Sk)) * 3)
        V, R = rng.normal(size=(Sk, H)), rng.normal(size=(S, H))
        X = rng.normal(size=(S, H)) * 4
        s = 1.0 / np.sqrt(H)
        ref = reference_ds(P, R, V, s)
        got = folded_ds(P, R, V, X, s)
        assert np.max(np.abs(got - ref)) <= 1e-12 * np.max(np.abs(ref))
        # dS rows sum to zero (softmax is shift invariant), both ways.
        assert np.max(np.abs(got.sum(axis=1))) <= 1e-12 * np.max(np.abs(ref))


def test_folded_softmax_backward_catches_slips():
    rng = np.random.default_rng(6)
    S, Sk, H = 32, 48, 16
    P = softmax64(rng.normal(size=(S, Sk)) * 3)
    V, R = rng.normal(size=(Sk, H)), rng.normal(size=(S, H))
    X = rng.normal(size=(S, H)) * 4
    s = 1.0 / np.sqrt(H)
    ref = reference_ds(P, R, V, s)
    scale = np.max(np.abs(ref))
    pre = P @ V + X
    dP = R @ V.T
    slips = {
        "residual kept": (R * pre).sum(axis=1, keepdims=True),
        "sum over rows": (R * (pre - X)).sum(axis=0, keepdims=True)[:, :1].repeat(S, 0),
        "no row sum": (R * (pre - X))[:, :1],
    }
    for name, D in slips.items():
        wrong = P * (s * dP - s * D)
        assert np.max(np.abs(wrong - ref)) > 1e-3 * scale, name
