"""Pins the f64 executor oracle (oracle/executors.py): every gradient by
central finite differences of its own forward at tiny shapes, and the
forward wiring by closed-form special cases (zero projections, uniform
attention, the 1/sqrt(d) score scale, residual placement)."""
import numpy as np
import pytest

from oracle import executors as ex


def rnd(seed, *shape, scale=0.5):
    return np.random.default_rng(seed).normal(0, scale, shape)


def params(S=4, H=4, F=6, O=3, seed=0, affine=True, bias=True):
    p = {"WQ": rnd(seed, H, H), "WK": rnd(seed + 1, H, H), "WV": rnd(seed + 2, H, H),
         "POS": rnd(seed + 3, S, H), "W1": rnd(seed + 4, H, F), "W2": rnd(seed + 5, F, H),
         "WO": rnd(seed + 6, H, O)}
    for k, n in (("BQ", H), ("BK", H), ("BV", H), ("B1", F), ("B2", H), ("BO", O)):
        p[k] = rnd(seed + 10 + len(k) + n, n, scale=0.1) if bias else None
    for k in ("G1", "G2"):
        p[k] = 1 + rnd(seed + 20 + len(k), H, scale=0.1) if affine else None
    for k in ("BE1", "BE2"):
        p[k] = rnd(seed + 30 + len(k), H, scale=0.1) if affine else None
    return p


def fd(f, x, h=1e-6):
    x = np.array(x, dtype=np.float64)
    g = np.zeros_like(x)
    for i in np.ndindex(x.shape):
        a, b = x.copy(), x.copy()
        a[i] += h
        b[i] -= h
        g[i] = (f(a) - f(b)) / (2 * h)
    return g


@pytest.mark.parametrize("norm_kind", [ex.LAYER, ex.RMS])
@pytest.mark.parametrize("ffn_act", [ex.GELU, ex.RELU, ex.SILU])
def test_transformer_gradients_finite_difference(norm_kind, ffn_act):
    S, H, F, O = 4, 4, 6, 3
    p = params(S, H, F, O, seed=norm_kind * 7 + ffn_act)
    if norm_kind == ex.RMS:
        p["BE1"] = p["BE2"] = None
    X = rnd(99, S, H)
    dY = rnd(98, S, O)

    def loss(pp, XX):
        out, _ = ex.transformer_forward(pp, XX, norm_kind, ffn_act)
        return float((out * dY).sum())

    _, cache = ex.transformer_forward(p, X, norm_kind, ffn_act)
    dX, g = ex.transformer_backward(p, cache, dY, norm_kind, ffn_act)
    # Xp = X + POS, so dX == dPOS
    assert np.allclose(dX, fd(lambda z: loss(p, z), X), atol=1e-6)
    assert np.allclose(g["POS"], dX)
    for k, v in p.items():
        if v is None or k == "POS":
            continue
        num = fd(lambda z: loss({**p, k: z}, X), v)
        assert g[k] is not None, k
        assert np.allclose(g[k], num, atol=1e-6), k


def test_zero_query_weights_give_uniform_attention():
    S, H = 5, 4
    p = params(S, H, 6, 3, seed=3)
    p["WQ"] = np.zeros((H, H))
    p["BQ"] = np.zeros(H)
    X = rnd(1, S, H)
    _, c = ex.transformer_forward(p, X, ex.LAYER)
    assert np.allclose(c["P"], 1.0 / S)
    assert np.allclose(c["pre1"], c["Xp"] + c["V"].mean(axis=0, keepdims=True))


def test_zero_value_weights_make_attention_a_pure_residual():
    p = params(4, 4, 6, 3, seed=4)
    p["WV"] = np.zeros((4, 4))
    p["BV"] = np.zeros(4)
    X = rnd(2, 4, 4)
    _, c = ex.transformer_forward(p, X, ex.RMS)
    assert np.allclose(c["pre1"], X + p["POS"])
    assert np.allclose(c["out1"], ex.norm_forward(X + p["POS"], ex.RMS, p["G1"]))


def test_zero_ffn_output_layer_adds_only_its_bias():
    p = params(4, 4, 6, 3, seed=5)
    p["W2"] = np.zeros((6, 4))
    X = rnd(3, 4, 4)
    _, c = ex.transformer_forward(p, X, ex.LAYER)
    assert np.allclose(c["pre2"], c["out1"] + p["B2"][None, :])


def test_score_scale_is_one_over_sqrt_query_width():
    # Xp rows a*e1, a*e2 with identity Q/K projections: scores a^2/sqrt(H) on
    # the diagonal and 0 elsewhere.
    H, a = 4, 1.5
    p = params(2, H, 6, 3, seed=6, bias=False)
    p["WQ"] = np.eye(H)
    p["WK"] = np.eye(H)
    p["POS"] = np.zeros((2, H))
    X = np.zeros((2, H))
    X[0, 0] = X[1, 1] = a
    _, c = ex.transformer_forward(p, X, ex.LAYER)
    s = a * a / np.sqrt(H)
    assert np.allclose(c["P"][0], [np.exp(s) / (np.exp(s) + 1), 1 / (np.exp(s) + 1)])


def test_causal_mask_zeroes_future_positions():
    p = params(5, 4, 6, 3, seed=7)
    _, c = ex.transformer_forward(p, rnd(4, 5, 4), ex.LAYER, causal=True)
    assert np.allclose(np.triu(c["P"], 1), 0)
    assert np.allclose(c["P"].sum(axis=1), 1)


@pytest.mark.parametrize("res_range", [None, (0, 2), (1, 3), (0, 3)])
def test_mlp_gradients_finite_difference(res_range):
    dims = [4, 5, 5, 4] if res_range else [4, 6, 5, 3]
    acts = [ex.GELU, ex.SILU, ex.IDENTITY]
    layers = [(rnd(10 + i, dims[i], dims[i + 1]), rnd(20 + i, dims[i + 1], scale=0.1), acts[i])
              for i in range(3)]
    if res_range == (0, 2):
        layers[1] = (rnd(31, 5, 4), layers[1][1][:4], acts[1])
        layers[2] = (rnd(32, 4, 4), layers[2][1], acts[2])
        dims = [4, 5, 4, 4]
    if res_range == (1, 3):
        dims = [4, 5, 5, 5]
        layers = [(rnd(40 + i, dims[i], dims[i + 1]), rnd(50 + i, dims[i + 1], scale=0.1), acts[i])
                  for i in range(3)]
    if res_range == (0, 3):
        dims = [4, 5, 5, 4]
        layers = [(rnd(60 + i, dims[i], dims[i + 1]), rnd(70 + i, dims[i + 1], scale=0.1), acts[i])
                  for i in range(3)]
    X = rnd(5, 3, dims[0])
    dY = rnd(6, 3, dims[-1])
    out, ins, pres = ex.mlp_forward(layers, X, res_range)
    dX, dWs, dbs = ex.mlp_backward(layers, ins, pres, dY, res_range)

    def loss(ls, XX):
        return float((ex.mlp_forward(ls, XX, res_range)[0] * dY).sum())

    assert np.allclose(dX, fd(lambda z: loss(layers, z), X), atol=1e-6)
    for i, (W, b, a) in enumerate(layers):
        numW = fd(lambda z: loss(layers[:i] + [(z, b, a)] + layers[i + 1:], X), W)
        numb = fd(lambda z: loss(layers[:i] + [(W, z, a)] + layers[i + 1:], X), b)
        assert np.allclose(dWs[i], numW, atol=1e-6)
        assert np.allclose(dbs[i], numb, atol=1e-6)


def test_loss_rows_closed_form():
    O = np.array([[1.0, 2.0], [3.0, 5.0]])
    T = np.array([[0.0, 0.0], [3.0, 3.0]])
    assert np.allclose(ex.loss_rows(O, T), [(0.5 + 2.0) / 2, (0 + 2.0) / 2])


@pytest.mark.parametrize("rms", [True, False])
def test_c_mirror_block_forward_matches_f64_executor(rms):
    """The C-kernel composition of the block forward (oracle.transformer_forward,
    timed by bench.py as the host baseline) equals the f64 executor oracle to
    f32 rounding: same wiring, same score scale, same activation."""
    from oracle import oracle as orc

    S, H, F, O = 24, 16, 40, 12
    p64 = params(S, H, F, O, seed=3, affine=False)
    p = {k: (None if v is None else v.astype(np.float32)) for k, v in p64.items()}
    X = rnd(9, S, H, scale=1.0).astype(np.float32)
    got = orc.transformer_forward(p, X, rms=rms)
    ref, _ = ex.transformer_forward(p, X, ex.RMS if rms else ex.LAYER)
    assert got.shape == (S, O)
    assert np.max(np.abs(got - ref)) <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("rms,affine,bias", [(False, True, True), (True, True, True),
                                             (False, False, True), (True, False, False)])
def test_c_mirror_training_step_matches_f64_executor(rms, affine, bias):
    """The C-kernel composition of the training step
    (oracle.transformer_training_step, timed by bench.py as the C5 host
    baseline) equals the f64 executor oracle to f32 rounding on the output,
    the input gradient and every parameter gradient, and each new parameter
    is the old one minus lr times its gradient with the reference's two
    roundings (scale, then subtract)."""
    from oracle import oracle as orc

    S, H, F, O = 24, 16, 40, 12
    p64 = params(S, H, F, O, seed=5, affine=affine, bias=bias)
    if rms:
        p64["BE1"] = p64["BE2"] = None
    p = {k: (None if v is None else v.astype(np.float32)) for k, v in p64.items()}
    X = rnd(11, S, H, scale=1.0).astype(np.float32)
    dY = rnd(12, S, O, scale=1.0).astype(np.float32)
    lr = np.float32(0.01)
    kind = ex.RMS if rms else ex.LAYER
    out, dx, grads, new = orc.transformer_training_step(p, X, dY, float(lr), rms=rms)
    ref, cache = ex.transformer_forward(p, X, kind)
    rdx, rg = ex.transformer_backward(p, cache, dY, kind)

    def close(a, b):
        return np.max(np.abs(a - b)) <= 1e-5 * max(1.0, np.abs(b).max())

    assert close(out, ref)
    assert close(dx, rdx)
    for k in p:
        if p[k] is None:
            assert grads.get(k) is None, k
            continue
        if k == "BK":
            # identically zero in exact arithmetic (softmax shift invariance)
            assert np.max(np.abs(grads[k])) <= 1e-5 * max(1.0, np.abs(rg["BV"]).max())
        else:
            assert close(grads[k], rg[k]), k
        assert np.array_equal(new[k], p[k] - lr * grads[k]), k
