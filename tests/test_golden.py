"""Golden known-answer vectors (tests/golden/*.npz, written by
tests/golden/make_golden.py from PyTorch float64 autograd) against the
oracle (CPU) and the HIP product (GPU, through the C ABI).

The fixtures come from an implementation independent of both the oracle and
the product: a forward pass written from the mathematics of the reference's
operators, with every gradient taken by autograd.  The oracle computes in
float64 and returns float32 for the kernel functions, so those agree to f32
rounding; its executors stay in float64 and agree to ~1e-12.  The product
is held to the same bars as its oracle parity tests.
"""
import os

import numpy as np
import pytest

from oracle import executors as ex
from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def rel(a, b):
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def absdiff(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


SLOTS = ex.SLOTS


def transformer_params(g, norm):
    p = {k: g["p_" + k] for k in SLOTS}
    if norm == "rms":
        p["BE1"] = p["BE2"] = None
    return p


# ------------------------------------------------------------- CPU oracle
F32 = 2e-7  # f32 rounding of an f64 result, relative to the largest entry


def test_oracle_gemm_golden():
    g = load("gemm")
    assert rel(orc.gemm(g["A"], g["B"]), g["C"]) <= F32
    assert rel(orc.gemm_f64(g["A"], g["B"]), g["C"]) <= 1e-14
    # Transposed operands stored transposed give the same product.
    At, Bt = np.ascontiguousarray(g["A"].T), np.ascontiguousarray(g["B"].T)
    assert rel(orc.gemm_f64(At, Bt, trans_a=True, trans_b=True), g["C"]) <= 1e-14


def test_oracle_rows_golden():
    g = load("rows")
    x, dy, gm, bt = g["x"], g["g"], g["gamma"], g["beta"]
    assert absdiff(orc.softmax_rows(x), g["softmax_y"]) <= 1e-7
    assert absdiff(orc.softmax_rows_backward(orc.softmax_rows(x), dy), g["softmax_dx"]) <= 1e-6
    assert absdiff(orc.layer_norm(x), g["ln_y"]) <= 1e-6
    assert absdiff(orc.layer_norm(x, gm, bt), g["ln_affine_y"]) <= 1e-6
    assert absdiff(orc.layer_norm_backward(x, dy), g["ln_dx"]) <= 1e-6
    dx, dgm, dbt = orc.layer_norm_backward(x, dy, gm, want_params=True)
    assert absdiff(dx, g["ln_affine_dx"]) <= 1e-6
    assert absdiff(dgm, g["ln_dgamma"]) <= 1e-6 and absdiff(dbt, g["ln_dbeta"]) <= 1e-6
    assert absdiff(orc.rms_norm(x), g["rms_y"]) <= 1e-6
    assert absdiff(orc.rms_norm(x, gm), g["rms_affine_y"]) <= 1e-6
    assert absdiff(orc.rms_norm_backward(x, dy), g["rms_dx"]) <= 1e-6
    dx, dgm = orc.rms_norm_backward(x, dy, gm, want_params=True)
    assert absdiff(dx, g["rms_affine_dx"]) <= 1e-6 and absdiff(dgm, g["rms_dgamma"]) <= 1e-6
    masked = orc.causal_mask(g["causal_x"])
    assert absdiff(orc.softmax_rows(masked), g["causal_softmax_y"]) <= 1e-7


def test_oracle_activations_golden():
    g = load("act")
    x = g["x"]
    for name, op, dop in (("gelu", orc.MAP_GELU, orc.MAP_GELU_D),
                          ("relu", orc.MAP_RELU, orc.MAP_RELU_D),
                          ("silu", orc.MAP_SILU, orc.MAP_SILU_D)):
        assert rel(orc.map_(x, op), g[name]) <= F32, name
        assert absdiff(orc.map_(x, dop), g[name + "_d"]) <= 1e-6, name + "'"
        a = {"gelu": ex.GELU, "relu": ex.RELU, "silu": ex.SILU}[name]
        assert absdiff(ex.act(x.astype(np.float64), a), g[name]) <= 1e-12
        assert absdiff(ex.act_d(x.astype(np.float64), a), g[name + "_d"]) <= 1e-12


def mlp_layers(g):
    acts = [ex.GELU, ex.SILU, ex.IDENTITY]
    return [(g[f"W{i}"], g[f"b{i}"], acts[i]) for i in range(3)]


def test_oracle_mlp_golden():
    g = load("mlp")
    res = tuple(int(v) for v in g["res"])
    layers = mlp_layers(g)
    y, ins, pres = ex.mlp_forward(layers, g["x"], res)
    assert rel(y, g["y"]) <= 1e-12
    dx, dWs, dbs = ex.mlp_backward(layers, ins, pres, g["dy"], res)
    assert rel(dx, g["dx"]) <= 1e-12
    for i in range(3):
        assert rel(dWs[i], g[f"dW{i}"]) <= 1e-12 and rel(dbs[i], g[f"db{i}"]) <= 1e-12


@pytest.mark.parametrize("norm", ["layer", "rms"])
def test_oracle_transformer_golden(norm):
    g = load("transformer")
    kind = ex.LAYER if norm == "layer" else ex.RMS
    p = transformer_params(g, norm)
    y, cache = ex.transformer_forward(p, g["x"], kind)
    assert rel(y, g[f"{norm}_y"]) <= 1e-12
    dx, grads = ex.transformer_backward(p, cache, g["dy"], kind)
    assert rel(dx, g[f"{norm}_dx"]) <= 1e-12
    scale = np.max(np.abs(g[f"{norm}_dBV"]))
    for k in SLOTS:
        if p.get(k) is None:
            continue
        if k == "BK":
            # Zero in exact arithmetic (softmax shift invariance); both sides
            # hold only rounding noise.
            assert np.max(np.abs(grads[k])) <= 1e-12 * scale
            assert np.max(np.abs(g[f"{norm}_dBK"])) <= 1e-12 * scale
            continue
        # POS enters as X + POS, so its gradient is dX.
        assert rel(grads[k], g[f"{norm}_d{k}"]) <= 1e-11, k


def test_oracle_transformer_causal_golden():
    g = load("transformer")
    y, _ = ex.transformer_forward(transformer_params(g, "layer"), g["x"], ex.LAYER, causal=True)
    assert rel(y, g["layer_causal_y"]) <= 1e-12


# ------------------------------------------------------------ GPU product
@pytest.mark.gpu
def test_gpu_gemm_golden(rt):
    g = load("gemm")
    M, K = g["A"].shape
    N = g["B"].shape[1]
    c = rt.empty((M, N))
    rt.gemm(rt.array(g["A"]), rt.array(g["B"]), c, M, N, K)
    assert rel(c.numpy(), g["C"]) <= 1e-4


@pytest.mark.gpu
def test_gpu_rows_golden(rt):
    g = load("rows")
    x, dy, gm, bt = g["x"], g["g"], g["gamma"], g["beta"]
    R, C = x.shape
    dgm, dbt = rt.array(gm), rt.array(bt)

    def fwd(fn, *extra):
        d = rt.array(x)
        fn(d, R, C, *extra)
        return d.numpy()

    assert absdiff(fwd(rt.softmax_rows), g["softmax_y"]) <= 1e-5
    assert absdiff(fwd(rt.layer_norm), g["ln_y"]) <= 1e-5
    assert absdiff(fwd(rt.layer_norm, dgm, dbt), g["ln_affine_y"]) <= 1e-5
    assert absdiff(fwd(rt.rms_norm), g["rms_y"]) <= 1e-5
    assert absdiff(fwd(rt.rms_norm, dgm), g["rms_affine_y"]) <= 1e-5

    p = rt.array(x)
    rt.softmax_rows(p, R, C)
    dx = rt.empty((R, C))
    rt.softmax_rows_bwd(p, rt.array(dy), dx, R, C)
    assert absdiff(dx.numpy(), g["softmax_dx"]) <= 1e-5

    ddg, ddb = rt.empty((C,)), rt.empty((C,))
    rt.layer_norm_bwd(rt.array(x), rt.array(dy), dx, R, C, dgm, ddg, ddb)
    assert absdiff(dx.numpy(), g["ln_affine_dx"]) <= 1e-5
    assert absdiff(ddg.numpy(), g["ln_dgamma"]) <= 1e-5
    assert absdiff(ddb.numpy(), g["ln_dbeta"]) <= 1e-5
    rt.rms_norm_bwd(rt.array(x), rt.array(dy), dx, R, C, dgm, ddg)
    assert absdiff(dx.numpy(), g["rms_affine_dx"]) <= 1e-5
    assert absdiff(ddg.numpy(), g["rms_dgamma"]) <= 1e-5

    m = rt.array(g["causal_x"])
    n = g["causal_x"].shape[0]
    rt.causal_mask(m, n, n)
    rt.softmax_rows(m, n, n)
    assert absdiff(m.numpy(), g["causal_softmax_y"]) <= 1e-5


@pytest.mark.gpu
def test_gpu_activations_golden(rt):
    import oxforge

    g = load("act")
    for name, op, dop in (("gelu", oxforge.MAP_GELU, oxforge.MAP_GELU_D),
                          ("relu", oxforge.MAP_RELU, oxforge.MAP_RELU_D),
                          ("silu", oxforge.MAP_SILU, oxforge.MAP_SILU_D)):
        for o, key in ((op, name), (dop, name + "_d")):
            d = rt.array(g["x"])
            rt.map(d, o)
            y = d.numpy()
            assert np.all(np.abs(y - g[key]) <= 2e-6 + 2e-6 * np.abs(g[key])), key


@pytest.mark.gpu
def test_gpu_mlp_golden(rt):
    from oxforge import net

    g = load("mlp")
    res = tuple(int(v) for v in g["res"])
    m = net.Mlp(rt, mlp_layers(g), res, training=True)
    y = m.forward(rt.array(g["x"])).numpy()
    assert rel(y, g["y"]) <= 1e-4
    lr = 1e-2
    dx = m.backward(rt.array(g["dy"]), lr).numpy()
    assert rel(dx, g["dx"]) <= 1e-4
    for i in range(3):
        assert rel(m.param(i, 0), g[f"W{i}"] - lr * g[f"dW{i}"]) <= 1e-4
        assert rel(m.param(i, 1), g[f"b{i}"] - lr * g[f"db{i}"]) <= 1e-4
    m.close()


@pytest.mark.gpu
@pytest.mark.parametrize("norm", ["layer", "rms"])
def test_gpu_transformer_golden(rt, norm):
    from oxforge import net

    g = load("transformer")
    S, H, F, O = (int(v) for v in g["dims"])
    p = transformer_params(g, norm)
    kind = net.LAYER if norm == "layer" else net.RMS
    T = net.Transformer(rt, p, S, H, F, O, kind, net.ENCODER_TRAINING)
    y = T.forward(rt.array(g["x"])).numpy()
    assert rel(y, g[f"{norm}_y"]) <= 1e-4
    dx = rt.empty((S, H))
    grads = T.backward(rt.array(g["dy"]), 1e-3, dx, want_grads=True)
    assert rel(dx.numpy(), g[f"{norm}_dx"]) <= 1e-4
    bad = {}
    for k in SLOTS:
        if p.get(k) is None:
            continue
        want = g[f"{norm}_d{k}"]
        got = grads[k].numpy()
        if k == "BK":
            # Exactly zero in exact arithmetic (softmax shift invariance):
            # bound the rounding noise against the value-bias gradient.
            err = float(np.max(np.abs(got)) / np.max(np.abs(g[f"{norm}_dBV"])))
        else:
            err = rel(got, want)
        if err > 1e-4:
            bad[k] = err
    assert not bad, bad
    T.close()


@pytest.mark.gpu
def test_gpu_decoder_golden(rt):
    from oxforge import net

    g = load("transformer")
    S, H, F, O = (int(v) for v in g["dims"])
    T = net.Transformer(rt, transformer_params(g, "layer"), S, H, F, O, net.LAYER,
                        net.DECODER_INFERENCE)
    y = T.forward(rt.array(g["x"])).numpy()
    assert rel(y, g["layer_causal_y"]) <= 1e-4
    T.close()
