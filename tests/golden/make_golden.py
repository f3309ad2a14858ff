"""Writes the golden fixtures in this directory (*.npz, no pickles).

The reference publishes no test vectors, and its arithmetic lives in an
un-vendored dependency (cuda-oxide) that cannot be built here.  These
fixtures are therefore known answers from an independent implementation:
PyTorch on the CPU in float64, with every gradient taken by autograd from a
forward pass written directly from the mathematics of the reference's
operators.  Neither the oracle nor the product is used to make them, so a
dropped term, a wrong sign or a transposed operand in either shows up as a
mismatch.

Inputs are drawn with numpy's PCG64 from fixed seeds and rounded to float32
(the value the device sees); outputs are float64.

Operators and the reference lines they follow:
  GEMM C = op(A) op(B)                     gemm.rs:202-373, matrix.rs:113-176
  softmax rows / backward                  row.rs:55-113, 193-237
  LayerNorm rows / backward (+gamma/beta)  row.rs:115-177, 239-347
  RMSNorm rows / backward (+gamma)         row.rs:349-468
  GELU (tanh form), ReLU, SiLU + d/dx      linear.rs:21-70
  causal mask before softmax               row.rs:5-14
  MLP with a residual range                mlp.rs:53-168
  single-head Post-Norm block, fwd + bwd   inference.rs:76-108, encoder.rs:114-186,
                                           attention.rs:221-401

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
EPS = float(np.float32(1e-5))             # norm.rs:45
GELU_SCALE = float(np.float32(0.7978846))  # linear.rs:22-24
GELU_CUBIC = float(np.float32(0.044715))

torch.set_default_dtype(torch.float64)


def f32(rng, shape, scale=1.0, loc=0.0):
    return (loc + scale * rng.standard_normal(shape)).astype(np.float32)


def t(a):
    return torch.tensor(np.asarray(a, np.float64))


def np64(x):
    return x.detach().numpy().astype(np.float64)


# ------------------------------------------------------------ operators
def gelu(x):
    return 0.5 * x * (1.0 + torch.tanh(GELU_SCALE * (x + GELU_CUBIC * x ** 3)))


def act(x, kind):
    return {"identity": lambda v: v, "gelu": gelu, "relu": torch.relu,
            "silu": lambda v: v * torch.sigmoid(v)}[kind](x)


def layer_norm(x, g=None, b=None):
    mu = x.mean(dim=1, keepdim=True)
    var = ((x - mu) ** 2).mean(dim=1, keepdim=True)
    y = (x - mu) / torch.sqrt(var + EPS)
    if g is not None:
        y = y * g
    if b is not None:
        y = y + b
    return y


def rms_norm(x, g=None):
    y = x / torch.sqrt((x * x).mean(dim=1, keepdim=True) + EPS)
    return y * g if g is not None else y


def grads(out, upstream, wrt):
    """Gradients of sum(out * upstream) with respect to each tensor in wrt."""
    gs = torch.autograd.grad((out * upstream).sum(), wrt, allow_unused=True)
    return [None if g is None else np64(g) for g in gs]


# ------------------------------------------------------------- fixtures
def make_gemm(rng):
    A, B = f32(rng, (7, 13)), f32(rng, (13, 5))
    return {"A": A, "B": B, "C": np64(t(A) @ t(B))}


def make_rows(rng):
    rows, cols = 6, 37
    x, g = f32(rng, (rows, cols), 2.0, 0.5), f32(rng, (rows, cols))
    gamma, beta = f32(rng, (cols,), 0.1, 1.0), f32(rng, (cols,), 0.1)
    out = {"x": x, "g": g, "gamma": gamma, "beta": beta}
    X = t(x).requires_grad_(True)
    Gm, Bt = t(gamma).requires_grad_(True), t(beta).requires_grad_(True)
    y = torch.softmax(X, dim=1)
    out["softmax_y"] = np64(y)
    out["softmax_dx"], = grads(y, t(g), [X])
    y = layer_norm(X)
    out["ln_y"] = np64(y)
    out["ln_dx"], = grads(y, t(g), [X])
    y = layer_norm(X, Gm, Bt)
    out["ln_affine_y"] = np64(y)
    out["ln_affine_dx"], out["ln_dgamma"], out["ln_dbeta"] = grads(y, t(g), [X, Gm, Bt])
    y = rms_norm(X)
    out["rms_y"] = np64(y)
    out["rms_dx"], = grads(y, t(g), [X])
    y = rms_norm(X, Gm)
    out["rms_affine_y"] = np64(y)
    out["rms_affine_dx"], out["rms_dgamma"] = grads(y, t(g), [X, Gm])
    # Causal softmax on a square block (masked entries are exactly zero).
    s = f32(rng, (9, 9))
    S = t(s).masked_fill(torch.triu(torch.ones(9, 9, dtype=torch.bool), 1), float("-inf"))
    out["causal_x"] = s
    out["causal_softmax_y"] = np64(torch.softmax(S, dim=1))
    return out


def make_act(rng):
    x = np.linspace(-6.0, 6.0, 97).astype(np.float32)
    x = x[x != 0.0]  # ReLU's derivative is a convention at 0
    out = {"x": x}
    for kind in ("gelu", "relu", "silu"):
        X = t(x).requires_grad_(True)
        y = act(X, kind)
        out[kind] = np64(y)
        out[kind + "_d"], = grads(y, torch.ones_like(y), [X])
    return out


def make_mlp(rng):
    dims, acts, res = [10, 14, 10, 8], ["gelu", "silu", "identity"], (0, 2)
    rows = 9
    x, dy = f32(rng, (rows, dims[0])), f32(rng, (rows, dims[-1]))
    out = {"x": x, "dy": dy, "res": np.array(res, np.int64)}
    W = [t(f32(rng, (dims[i], dims[i + 1]), 0.4)).requires_grad_(True) for i in range(3)]
    b = [t(f32(rng, (dims[i + 1],), 0.1)).requires_grad_(True) for i in range(3)]
    for i in range(3):
        out[f"W{i}"], out[f"b{i}"] = W[i].detach().numpy().astype(np.float32), \
            b[i].detach().numpy().astype(np.float32)
    X = t(x).requires_grad_(True)
    inputs, cur = [X], X
    for i in range(3):
        z = cur @ W[i] + b[i]
        if i + 1 == res[1]:
            z = z + inputs[res[0]]
        cur = act(z, acts[i])
        inputs.append(cur)
    out["y"] = np64(cur)
    gs = grads(cur, t(dy), [X] + W + b)
    out["dx"] = gs[0]
    for i in range(3):
        out[f"dW{i}"], out[f"db{i}"] = gs[1 + i], gs[4 + i]
    return out


SLOTS = ["WQ", "BQ", "WK", "BK", "WV", "BV", "POS", "W1", "B1", "W2", "B2", "WO", "BO",
         "G1", "BE1", "G2", "BE2"]


def block_forward(p, X, norm, causal):
    """Post-Norm single-head block: attention + residual + norm, FFN (GELU)
    + residual + norm, output projection."""
    Xp = X + p["POS"]
    Q = Xp @ p["WQ"] + p["BQ"]
    K = Xp @ p["WK"] + p["BK"]
    V = Xp @ p["WV"] + p["BV"]
    S = (Q @ K.T) * (1.0 / np.sqrt(np.float32(Q.shape[1])))
    if causal:
        n = S.shape[0]
        S = S.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool), 1), float("-inf"))
    P = torch.softmax(S, dim=1)
    pre1 = Xp + P @ V
    nrm = (lambda x, g, b: layer_norm(x, g, b)) if norm == "layer" else \
        (lambda x, g, b: rms_norm(x, g))
    out1 = nrm(pre1, p["G1"], p.get("BE1"))
    H1 = gelu(out1 @ p["W1"] + p["B1"])
    pre2 = out1 + (H1 @ p["W2"] + p["B2"])
    enc = nrm(pre2, p["G2"], p.get("BE2"))
    return enc @ p["WO"] + p["BO"]


def make_transformer(rng):
    S, H, F, O = 8, 16, 32, 12
    out = {"dims": np.array([S, H, F, O], np.int64)}
    shapes = {"WQ": (H, H), "BQ": (H,), "WK": (H, H), "BK": (H,), "WV": (H, H), "BV": (H,),
              "POS": (S, H), "W1": (H, F), "B1": (F,), "W2": (F, H), "B2": (H,),
              "WO": (H, O), "BO": (O,), "G1": (H,), "BE1": (H,), "G2": (H,), "BE2": (H,)}
    host = {}
    for k in SLOTS:
        if k.startswith("G"):
            host[k] = f32(rng, shapes[k], 0.1, 1.0)
        elif k.startswith("B"):
            host[k] = f32(rng, shapes[k], 0.1)
        else:
            host[k] = f32(rng, shapes[k], 1.0 / np.sqrt(shapes[k][0]))
        out["p_" + k] = host[k]
    x, dy = f32(rng, (S, H)), f32(rng, (S, O))
    out["x"], out["dy"] = x, dy
    for norm in ("layer", "rms"):
        p = {k: t(v).requires_grad_(True) for k, v in host.items()
             if not (norm == "rms" and k in ("BE1", "BE2"))}
        X = t(x).requires_grad_(True)
        Y = block_forward(p, X, norm, causal=False)
        out[f"{norm}_y"] = np64(Y)
        names = list(p)
        gs = grads(Y, t(dy), [X] + [p[k] for k in names])
        out[f"{norm}_dx"] = gs[0]
        for k, g in zip(names, gs[1:]):
            out[f"{norm}_d{k}"] = g
    p = {k: t(v) for k, v in host.items()}
    out["layer_causal_y"] = np64(block_forward(p, t(x), "layer", causal=True))
    return out


def main():
    makers = {"gemm": make_gemm, "rows": make_rows, "act": make_act, "mlp": make_mlp,
              "transformer": make_transformer}
    for i, (name, fn) in enumerate(makers.items()):
        data = fn(np.random.default_rng(1000 + i))
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **data)
        print(f"{path}: {len(data)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
