"""f64 numpy restatement of the OxideForge executors (Linear, MLP, Attention,
single-head Post-Norm transformer, forward and backward with SGD).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP executors (the
product never imports this).  Everything is evaluated in float64 from f32
inputs, i.e. the exact mathematics of the reference's algorithm; pinned by
central finite differences and closed-form special cases in
tests/test_oracle_executors.py, and to 1e-11 by the PyTorch float64
autograd known answers of tests/golden/ (tests/test_golden.py).  Reference
files are under src/net/.
"""
from __future__ import annotations

import numpy as np

# Activation constants, as the f32 values the reference uses (linear.rs:22-24).
GELU_SCALE = float(np.float32(0.7978846))
GELU_CUBIC = float(np.float32(0.044715))
EPS = float(np.float32(1e-5))  # norm.rs:45,66,123,153

IDENTITY, GELU, RELU, SILU = 0, 1, 2, 3
RMS, LAYER = 0, 1


def act(x, a):
    """Activation::forward (linear.rs:26-43)."""
    if a == GELU:
        return 0.5 * x * (1.0 + np.tanh(GELU_SCALE * (x + GELU_CUBIC * x ** 3)))
    if a == RELU:
        return np.where(x > 0, x, 0.0)
    if a == SILU:
        return x / (1.0 + np.exp(-x))
    return x


def act_d(x, a):
    """Activation::derivative (linear.rs:45-69)."""
    if a == GELU:
        t = np.tanh(GELU_SCALE * (x + GELU_CUBIC * x ** 3))
        return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * (GELU_SCALE + 3 * GELU_SCALE * GELU_CUBIC * x * x)
    if a == RELU:
        return (x > 0).astype(np.float64)
    if a == SILU:
        e = np.exp(-x)
        return 1 / (1 + e) + x * e / ((1 + e) * (1 + e))
    return np.ones_like(x)


def f64(a):
    return None if a is None else np.asarray(a, dtype=np.float64)


# --------------------------------------------------------------- Linear
def linear_forward(X, W, b=None, R=None, a=IDENTITY):
    """Linear::forward (linear.rs:116-230): Z = X W (+ b by rows) (+ R);
    returns (act(Z), Z)."""
    Z = f64(X) @ f64(W)
    if b is not None:
        Z = Z + f64(b)[None, :]
    if R is not None:
        Z = Z + f64(R)
    return act(Z, a), Z


def linear_backward(Z, dY, a, has_bias):
    """Linear::backward (linear.rs:232-306): G = dY * act'(Z), db = sum_rows G."""
    G = f64(dY) * act_d(f64(Z), a)
    return G, (G.sum(axis=0) if has_bias else None)


def loss_rows(O, T):
    """Linear::loss_rows (linear.rs:312-348)."""
    d = f64(O) - f64(T)
    return (0.5 * d * d).sum(axis=1) / d.shape[1]


# ----------------------------------------------------------------- norms
def norm_forward(x, kind, g=None, b=None, eps=EPS):
    """LayerNorm (row.rs:115-177) / RMSNorm (row.rs:349-396) + affine ext."""
    x = f64(x)
    if kind == LAYER:
        mu = x.mean(axis=1, keepdims=True)
        y = (x - mu) / np.sqrt(((x - mu) ** 2).mean(axis=1, keepdims=True) + eps)
        if g is not None:
            y = y * f64(g)
        if b is not None:
            y = y + f64(b)
        return y
    y = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps)
    return y * f64(g) if g is not None else y


def norm_backward(x, dy, kind, g=None, eps=EPS):
    """LN backward (row.rs:239-347) / RMS backward (row.rs:398-468) with the
    affine extension; returns (dx, dgamma, dbeta)."""
    x, dy = f64(x), f64(dy)
    n = x.shape[1]
    gg = dy * f64(g) if g is not None else dy
    if kind == LAYER:
        mu = x.mean(axis=1, keepdims=True)
        r = 1 / np.sqrt(((x - mu) ** 2).mean(axis=1, keepdims=True) + eps)
        xh = (x - mu) * r
        A = gg.sum(axis=1, keepdims=True)
        B = (gg * xh).sum(axis=1, keepdims=True)
        dx = r / n * (n * gg - A - xh * B)
        return dx, (dy * xh).sum(axis=0), dy.sum(axis=0)
    inv = 1 / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps)
    d = (x * gg).sum(axis=1, keepdims=True)
    dx = gg * inv - x * (d / n * inv ** 3)
    return dx, (dy * x * inv).sum(axis=0), None


def softmax(x):
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


# ------------------------------------------------------------ transformer
SLOTS = ["WQ", "BQ", "WK", "BK", "WV", "BV", "POS", "W1", "B1", "W2", "B2", "WO", "BO",
         "G1", "BE1", "G2", "BE2"]


def transformer_forward(p, X, norm_kind, ffn_act=GELU, causal=False):
    """encoder/decoder forward (inference.rs:76-108, encoder.rs:114-131,
    attention.rs:258-281, 359-401).  p maps slot names to arrays (biases and
    G*/BE* may be None).  Returns (output, cache)."""
    Xp = f64(X) + f64(p["POS"])
    Q, _ = linear_forward(Xp, p["WQ"], p.get("BQ"))
    K, _ = linear_forward(Xp, p["WK"], p.get("BK"))
    V, _ = linear_forward(Xp, p["WV"], p.get("BV"))
    S = (Q @ K.T) * (1.0 / np.sqrt(np.float32(Q.shape[1])))
    if causal:
        S = np.where(np.arange(S.shape[1])[None, :] > np.arange(S.shape[0])[:, None], -np.inf, S)
    P = softmax(S)
    pre1 = Xp + P @ V
    out1 = norm_forward(pre1, norm_kind, p.get("G1"), p.get("BE1"))
    H1, Z1 = linear_forward(out1, p["W1"], p.get("B1"), a=ffn_act)
    F2, _ = linear_forward(H1, p["W2"], p.get("B2"))
    pre2 = out1 + F2
    enc = norm_forward(pre2, norm_kind, p.get("G2"), p.get("BE2"))
    out, _ = linear_forward(enc, p["WO"], p.get("BO"))
    cache = dict(Xp=Xp, Q=Q, K=K, V=V, P=P, pre1=pre1, out1=out1, H1=H1, Z1=Z1, pre2=pre2,
                 enc=enc)
    return out, cache


def transformer_backward(p, cache, dY, norm_kind, ffn_act=GELU):
    """TrainingTransformer::backward (encoder.rs:133-186) without the SGD
    step: returns (dX, grads) with grads keyed like p (gradients of the
    parameters before their update)."""
    c = cache
    g = {}
    dY = f64(dY)
    # Output projection (identity activation).
    g["WO"] = c["enc"].T @ dY
    g["BO"] = dY.sum(axis=0) if p.get("BO") is not None else None
    d_enc = dY @ f64(p["WO"]).T
    d_pre2, g["G2"], g["BE2"] = norm_backward(c["pre2"], d_enc, norm_kind, p.get("G2"))
    # FFN (mlp.rs:121-168): layer 2 identity, layer 1 ffn_act.
    g["W2"] = c["H1"].T @ d_pre2
    g["B2"] = d_pre2.sum(axis=0) if p.get("B2") is not None else None
    dH1 = d_pre2 @ f64(p["W2"]).T
    G1 = dH1 * act_d(c["Z1"], ffn_act)
    g["W1"] = c["out1"].T @ G1
    g["B1"] = G1.sum(axis=0) if p.get("B1") is not None else None
    d_out1 = d_pre2 + G1 @ f64(p["W1"]).T
    # Attention (attention.rs:283-321 and 104-144).
    R, g["G1"], g["BE1"] = norm_backward(c["pre1"], d_out1, norm_kind, p.get("G1"))
    dP = R @ c["V"].T
    dV = c["P"].T @ R
    s = (dP * c["P"]).sum(axis=1, keepdims=True)
    dS = c["P"] * (dP - s) * (1.0 / np.sqrt(np.float32(c["Q"].shape[1])))
    dQ = dS @ c["K"]
    dK = dS.T @ c["Q"]
    proj = np.zeros_like(c["Xp"])
    for w, b, G in (("WQ", "BQ", dQ), ("WK", "BK", dK), ("WV", "BV", dV)):
        g[w] = c["Xp"].T @ G
        g[b] = G.sum(axis=0) if p.get(b) is not None else None
        proj = proj + G @ f64(p[w]).T
    dXp = R + proj
    g["POS"] = dXp
    if norm_kind == RMS:
        g["BE1"] = g["BE2"] = None
    if p.get("G1") is None:
        g["G1"] = g["BE1"] = None
    if p.get("G2") is None:
        g["G2"] = g["BE2"] = None
    return dXp, g


def sgd(p, grads, lr):
    """Linear::learn / position update: P -= lr * dP for every parameter."""
    return {k: (None if v is None else f64(v) - lr * grads[k]) for k, v in p.items()}


# ----------------------------------------------------------------- MLP
def mlp_forward(layers, X, res_range=None):
    """MlpExecutor::forward (mlp.rs:53-85); layers = [(W, b, act), ...].
    Returns (output, layer_inputs, pre_activations)."""
    inputs, pres = [f64(X)], []
    cur = f64(X)
    for i, (W, b, a) in enumerate(layers):
        R = inputs[res_range[0]] if res_range and i + 1 == res_range[1] else None
        cur, Z = linear_forward(cur, W, b, R, a)
        pres.append(Z)
        if i + 1 < len(layers):
            inputs.append(cur)
    return cur, inputs, pres


def mlp_backward(layers, inputs, pres, dY, res_range=None):
    """MlpExecutor::backward (mlp.rs:121-168) gradients; returns (dX, dWs, dbs)."""
    L = len(layers)
    dWs, dbs = [None] * L, [None] * L
    grad = f64(dY)
    skip = None
    for i in reversed(range(L)):
        W, b, a = layers[i]
        G, db = linear_backward(pres[i], grad, a, b is not None)
        dX = G @ f64(W).T
        if res_range and i + 1 == res_range[1]:
            skip = (res_range[0], G.copy())
        if skip and skip[0] == i:
            dX = dX + skip[1]
            skip = None
        dWs[i], dbs[i] = inputs[i].T @ G, db
        grad = dX
    return grad, dWs, dbs
