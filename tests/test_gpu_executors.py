"""GPU parity of the executors (Linear, MLP, transformer inference and
training step) against the f64 executor oracle (oracle/executors.py).

Bar: max|GPU - oracle| / max|oracle| <= 1e-4 for every output, input
gradient and parameter gradient (the GEMM/attention bound, applied to the
whole composition); the SGD update is checked bit-exactly as
W_new == fl(W - fl(lr * dW)) from the returned f32 gradient.
"""
import numpy as np
import pytest

import oxforge
from oracle import executors as ex
from oracle import oracle as orc
from oxforge import net
from oxforge import synth

pytestmark = pytest.mark.gpu
TOL = 1e-4


def say(msg):
    print(f"[case] {msg}", flush=True)


def rel(a, b):
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def make_params(S, H, F, O, seed, bias=True, affine=True, norm=net.LAYER):
    p = {"WQ": synth.xavier(H, H, seed), "WK": synth.xavier(H, H, seed + 1),
         "WV": synth.xavier(H, H, seed + 2), "POS": synth.xavier(S, H, seed + 3),
         "W1": synth.xavier(H, F, seed + 4), "W2": synth.xavier(F, H, seed + 5),
         "WO": synth.xavier(H, O, seed + 6)}
    for i, (k, n) in enumerate((("BQ", H), ("BK", H), ("BV", H), ("B1", F), ("B2", H), ("BO", O))):
        p[k] = synth.normal((n,), seed + 10 + i, 0.0, 0.1) if bias else None
    p["G1"] = synth.normal((H,), seed + 20, 1.0, 0.1) if affine else None
    p["G2"] = synth.normal((H,), seed + 21, 1.0, 0.1) if affine else None
    p["BE1"] = synth.normal((H,), seed + 22, 0.0, 0.1) if affine and norm == net.LAYER else None
    p["BE2"] = synth.normal((H,), seed + 23, 0.0, 0.1) if affine and norm == net.LAYER else None
    return p


# ------------------------------------------------------------------ Linear
def test_linear_c1_identity_no_bias(rt):
    """X [256,128] x W [128,64], identity, no bias."""
    say("linear C1")
    X = synth.uniform((256, 128), 1)
    W = synth.uniform((128, 64), 2)
    lin = net.Linear(rt, W)
    Y = lin.forward(rt.array(X)).numpy()
    ref, _ = ex.linear_forward(X, W)
    assert rel(Y, ref) <= TOL


@pytest.mark.parametrize("act", [0, 1, 2, 3])
def test_linear_forward_backward_learn(rt, act):
    say(f"linear act={act}")
    M, I, O = 96, 80, 48
    X, W = synth.uniform((M, I), 3), synth.uniform((I, O), 4)
    b, R = synth.uniform((O,), 5), synth.uniform((M, O), 6)
    dY = synth.normal((M, O), 7)
    lin = net.Linear(rt, W, b, act)
    dX_, dR = rt.array(X), rt.array(R)
    pre = rt.empty((M, O))
    Y = lin.forward(dX_, dR, pre_out=pre).numpy()
    refY, refZ = ex.linear_forward(X, W, b, R, act)
    assert rel(Y, refY) <= TOL and rel(pre.numpy(), refZ) <= TOL
    G, db = rt.empty((M, O)), rt.empty((O,))
    lin.backward(pre, rt.array(dY), G, db)
    refG, refdb = ex.linear_backward(pre.numpy(), dY, act, True)
    assert rel(G.numpy(), refG) <= TOL and rel(db.numpy(), refdb) <= TOL
    dXg = rt.empty((M, I))
    lin.input_gradient(G, dXg)
    assert rel(dXg.numpy(), G.numpy().astype(np.float64) @ W.T.astype(np.float64)) <= TOL
    lr = 1e-2
    lin.learn(dX_, G, db, lr)
    dW = X.T.astype(np.float64) @ G.numpy().astype(np.float64)
    assert rel(lin.param(0), W - lr * dW) <= TOL
    assert np.array_equal(lin.param(1), b - np.float32(lr) * db.numpy())


def test_loss_rows(rt):
    O, T = synth.normal((37, 21), 1), synth.normal((37, 21), 2)
    out = rt.empty((37,))
    net.loss_rows(rt, rt.array(O), rt.array(T), out)
    assert rel(out.numpy(), ex.loss_rows(O, T)) <= 1e-5


# --------------------------------------------------------------------- MLP
@pytest.mark.parametrize("res_range", [None, (0, 2), (1, 3), (0, 3)])
def test_mlp_training(rt, res_range):
    say(f"mlp res_range={res_range}")
    dims = {None: [64, 96, 80, 48], (0, 2): [64, 96, 64, 48], (1, 3): [64, 96, 80, 96],
            (0, 3): [64, 96, 80, 64]}[res_range]
    acts = [1, 3, 0]
    layers = [(synth.xavier(dims[i], dims[i + 1], 10 + i), synth.normal((dims[i + 1],), 20 + i, 0, 0.1),
               acts[i]) for i in range(3)]
    X, dY = synth.normal((50, dims[0]), 1), synth.normal((50, dims[-1]), 2)
    m = net.Mlp(rt, layers, res_range, training=True)
    Y = m.forward(rt.array(X)).numpy()
    ref, ins, pres = ex.mlp_forward(layers, X, res_range)
    assert rel(Y, ref) <= TOL
    lr = 1e-2
    dX = m.backward(rt.array(dY), lr).numpy()
    rdX, dWs, dbs = ex.mlp_backward(layers, ins, pres, dY, res_range)
    assert rel(dX, rdX) <= TOL
    for i, (W, b, _) in enumerate(layers):
        assert rel(m.param(i, 0), W - lr * dWs[i]) <= TOL
        assert rel(m.param(i, 1), b - lr * dbs[i]) <= TOL


# ------------------------------------------------------------- transformer
INFER_CASES = [
    ("encoder rms small", 64, 64, 256, 64, net.RMS, net.ENCODER_INFERENCE, True),
    ("encoder layer small", 96, 128, 256, 80, net.LAYER, net.ENCODER_INFERENCE, False),
    ("decoder layer small", 64, 64, 128, 32, net.LAYER, net.DECODER_INFERENCE, True),
    ("C4 full: S=2048 H=1024 F=4096 O=1024 RMS", 2048, 1024, 4096, 1024, net.RMS,
     net.ENCODER_INFERENCE, True),
]


@pytest.mark.parametrize("name,S,H,F,O,norm,kind,streams", INFER_CASES)
def test_transformer_inference(rt, name, S, H, F, O, norm, kind, streams):
    say(f"inference {name}")
    full = S == 2048
    p = make_params(S, H, F, O, 40, bias=not full, affine=not full, norm=norm)
    if full:  # biases zero, reference (parameterless) norm
        for k in ("BQ", "BK", "BV", "B1", "B2", "BO"):
            n = {"B1": F, "BO": O}.get(k, H)
            p[k] = np.zeros(n, np.float32)
    X = synth.normal((S, H), 4)
    T = net.Transformer(rt, p, S, H, F, O, norm, kind, streams)
    Y1 = T.forward(rt.array(X)).numpy()
    Y2 = T.forward(rt.array(X)).numpy()
    assert np.array_equal(Y1, Y2), "forward is not deterministic"
    ref, _ = ex.transformer_forward(p, X, norm, causal=(kind == net.DECODER_INFERENCE))
    err = rel(Y1, ref)
    print(f"  rel err {err:.3e}")
    assert err <= TOL


FOLD_CASES = [
    # (S, H, F, O, kind, score_bytes: None = unchunked)
    (128, 128, 256, 96, net.ENCODER_INFERENCE, None),
    (128, 128, 256, 96, net.DECODER_INFERENCE, None),
    (320, 256, 512, 128, net.DECODER_INFERENCE, 64 * 320 * 4),  # chunked attention
    (70, 48, 100, 36, net.ENCODER_INFERENCE, None),             # guarded tiles
    (2048, 1024, 4096, 1024, net.ENCODER_INFERENCE, None),      # C4
]


@pytest.mark.parametrize("S,H,F,O,kind,score_bytes", FOLD_CASES)
def test_rms_norms_folded_into_products(rt, S, H, F, O, kind, score_bytes):
    """With the reference's parameterless RMSNorms the inference block folds
    both norms into the products beside them (InferenceBlock::
    set_fold_norms, inference.rs:76-108 with norm.rs:50-69).  The folded
    forward matches the f64 oracle (1e-4) and the reference-ordered forward
    (the same kernels without the fold) to 1e-5 relative; the reference
    order is still selectable and still matches the oracle.  Covers
    encoder and decoder, query-chunked attention (the rows' statistics
    written per chunk) and odd sizes (the guarded tiles, whose statistics
    come from separate passes)."""
    say(f"folded RMSNorms S={S} H={H} F={F} O={O} kind={kind} chunked={score_bytes}")
    full = S == 2048
    p = make_params(S, H, F, O, 44, bias=not full, affine=False, norm=net.RMS)
    if full:
        for k, n in (("BQ", H), ("BK", H), ("BV", H), ("B1", F), ("B2", H), ("BO", O)):
            p[k] = np.zeros(n, np.float32)
    X = synth.normal((S, H), 6)
    Tf = net.Transformer(rt, p, S, H, F, O, net.RMS, kind)
    Tr = net.Transformer(rt, p, S, H, F, O, net.RMS, kind)
    Tr.set_fold_norms(False)
    if score_bytes:
        Tf.set_score_bytes(score_bytes)
        Tr.set_score_bytes(score_bytes)
    dX = rt.array(X)
    yf, yr = Tf.forward(dX).numpy(), Tr.forward(dX).numpy()
    Tf.close()
    Tr.close()
    ref, _ = ex.transformer_forward(p, X, net.RMS, causal=(kind == net.DECODER_INFERENCE))
    ef, er, d = rel(yf, ref), rel(yr, ref), rel(yf, yr)
    print(f"  folded {ef:.2e}, reference order {er:.2e}, folded vs reference order {d:.2e}")
    assert ef <= TOL and er <= TOL and d <= 1e-5


def test_fold_norms_leaves_other_norms_in_reference_order(rt):
    """The fold applies only to parameterless RMSNorms: with gamma, or with
    LayerNorm, the forward is the reference-ordered one bit for bit whatever
    the setting; the training kind refuses the setting."""
    S, H, F, O = 64, 64, 128, 48
    for norm, affine in ((net.RMS, True), (net.LAYER, False)):
        say(f"fold setting with norm={norm} affine={affine}")
        p = make_params(S, H, F, O, 45, bias=True, affine=affine, norm=norm)
        X = rt.array(synth.normal((S, H), 7))
        Ta = net.Transformer(rt, p, S, H, F, O, norm, net.ENCODER_INFERENCE)
        Tb = net.Transformer(rt, p, S, H, F, O, norm, net.ENCODER_INFERENCE)
        Tb.set_fold_norms(False)
        assert np.array_equal(Ta.forward(X).numpy(), Tb.forward(X).numpy())
        Ta.close()
        Tb.close()
    p = make_params(S, H, F, O, 46, bias=True, affine=False, norm=net.RMS)
    Tt = net.Transformer(rt, p, S, H, F, O, net.RMS, net.ENCODER_TRAINING)
    with pytest.raises(oxforge.ForgeError):
        Tt.set_fold_norms(True)
    Tt.close()


@pytest.mark.parametrize("S,H,F,O,kind", [(64, 64, 256, 64, net.ENCODER_INFERENCE),
                                           (96, 128, 256, 80, net.DECODER_INFERENCE),
                                           (2048, 1024, 4096, 1024, net.ENCODER_INFERENCE)])
def test_qkv_forked_streams_match_batched_bit_exact(rt, S, H, F, O, kind):
    """qkv_streams=1 runs Q, K and V on three forked streams joined before the
    scores and before A.V (attention.rs:65-102); qkv_streams=0 runs them as
    one batched launch.  Same products in the same sum order: bit-identical,
    on repeated forwards too (the second fork reuses the same streams)."""
    say(f"qkv streams vs batched S={S} H={H} kind={kind}")
    p = make_params(S, H, F, O, 41, bias=True, affine=True, norm=net.LAYER)
    X = synth.normal((S, H), 5)
    Ts = net.Transformer(rt, p, S, H, F, O, net.LAYER, kind, True)
    Tb = net.Transformer(rt, p, S, H, F, O, net.LAYER, kind, False)
    dX = rt.array(X)
    outs = [Ts.forward(dX).numpy(), Ts.forward(dX).numpy(), Tb.forward(dX).numpy()]
    assert np.array_equal(outs[0], outs[2]) and np.array_equal(outs[1], outs[2])
    ref, _ = ex.transformer_forward(p, X, net.LAYER, causal=(kind == net.DECODER_INFERENCE))
    assert rel(outs[0], ref) <= TOL
    Ts.close()
    Tb.close()


@pytest.mark.parametrize("kind", [net.ENCODER_INFERENCE, net.DECODER_INFERENCE])
@pytest.mark.parametrize("chunk_rows", [64, 128])
def test_query_chunked_attention_forward(rt, kind, chunk_rows):
    """With a score budget below seq x seq, attention runs one chunk of
    query rows at a time (320 rows: five chunks of 64, or 128 + 128 + 64; the
    decoder's causal mask offset per chunk).  Each output row is the same
    sequence of rounded operations as unchunked, so the forward is
    bit-identical to the unchunked one, and matches the f64 oracle."""
    S, H, F, O = 320, 64, 128, 48
    say(f"chunked attention forward kind={kind} chunk={chunk_rows}")
    p = make_params(S, H, F, O, 42, bias=True, affine=True, norm=net.LAYER)
    X = synth.normal((S, H), 9)
    Tc = net.Transformer(rt, p, S, H, F, O, net.LAYER, kind)
    Tu = net.Transformer(rt, p, S, H, F, O, net.LAYER, kind)
    Tc.set_score_bytes(chunk_rows * S * 4)
    dX = rt.array(X)
    yc, yu = Tc.forward(dX).numpy(), Tu.forward(dX).numpy()
    assert np.array_equal(yc, yu)
    ref, _ = ex.transformer_forward(p, X, net.LAYER, causal=(kind == net.DECODER_INFERENCE))
    assert rel(yc, ref) <= TOL
    Tc.close()
    Tu.close()


def test_query_chunked_attention_forward_with_split_products(rt):
    """S = Sk = 8192 in chunks of 64 query rows: each chunk's P V ([64, 8192]
    by [8192, 64], one output tile) is computed as K slices, the whole
    product is not, so the chunked forward agrees with the unchunked one to
    within rounding (1e-5 relative) rather than bit for bit, and matches the
    f64 oracle (1e-4)."""
    S, H, F, O = 8192, 64, 128, 48
    say(f"chunked attention forward S={S} chunk=64 (split P.V)")
    assert "split" in rt.gemm_kernel_name(64, H, S, fused=True)
    assert "split" not in rt.gemm_kernel_name(S, H, S, fused=True)
    p = make_params(S, H, F, O, 44, bias=True, affine=True, norm=net.LAYER)
    X = synth.normal((S, H), 12)
    Tc = net.Transformer(rt, p, S, H, F, O, net.LAYER, net.ENCODER_INFERENCE)
    Tu = net.Transformer(rt, p, S, H, F, O, net.LAYER, net.ENCODER_INFERENCE)
    Tc.set_score_bytes(64 * S * 4)
    dX = rt.array(X)
    yc, yu = Tc.forward(dX).numpy(), Tu.forward(dX).numpy()
    Tc.close()
    Tu.close()
    assert rel(yc, yu) <= 1e-5
    ref, _ = ex.transformer_forward(p, X, net.LAYER)
    assert rel(yc, ref) <= TOL


@pytest.mark.parametrize("S,chunk_rows,norm", [(320, 64, net.LAYER), (320, 128, net.LAYER),
                                              (512, 192, net.LAYER), (320, 64, net.RMS)])
def test_query_chunked_attention_training_step(rt, S, chunk_rows, norm):
    """Training with the score budget below seq x seq: the forward keeps no
    probabilities and backward recomputes them per chunk (dV and dK summed
    over the chunks in order; each chunk's dS formed in its dP product from
    the row term the norm backward wrote for all rows).  The forward output
    is bit-identical to the unchunked step; dX and every parameter gradient
    match the f64 oracle, and the unchunked step's to within 1e-5
    relative."""
    H, F, O = 64, 128, 48
    say(f"chunked attention training S={S} chunk={chunk_rows} norm={norm}")
    p = make_params(S, H, F, O, 43, bias=True, affine=True, norm=norm)
    X = synth.normal((S, H), 10)
    dY = synth.normal((S, O), 11)
    lr = 1e-3
    Tc = net.Transformer(rt, p, S, H, F, O, norm, net.ENCODER_TRAINING)
    Tu = net.Transformer(rt, p, S, H, F, O, norm, net.ENCODER_TRAINING)
    Tc.set_score_bytes(chunk_rows * S * 4)
    yc, yu = Tc.forward(rt.array(X)).numpy(), Tu.forward(rt.array(X)).numpy()
    assert np.array_equal(yc, yu)
    dxc, dxu = rt.empty((S, H)), rt.empty((S, H))
    gc = Tc.backward(rt.array(dY), lr, dxc, want_grads=True)
    gu = Tu.backward(rt.array(dY), lr, dxu, want_grads=True)
    _, cache = ex.transformer_forward(p, X, norm)
    rdX, rg = ex.transformer_backward(p, cache, dY, norm)
    assert rel(dxc.numpy(), rdX) <= TOL
    assert rel(dxc.numpy(), dxu.numpy()) <= 1e-5
    for k in net.TP_SLOTS:
        if rg.get(k) is None or p.get(k) is None:
            continue
        g = gc[k].numpy()
        if k == "BK":
            assert np.max(np.abs(g)) / np.max(np.abs(rg["BV"])) <= TOL
            continue
        assert rel(g, rg[k]) <= TOL, k
        assert rel(g, gu[k].numpy()) <= 1e-5, k
    Tc.close()
    Tu.close()


TRAIN_CASES = [
    ("layer small", 64, 64, 256, 64, net.LAYER, True, True),
    ("rms small no-bias", 48, 32, 96, 40, net.RMS, False, True),
    ("layer medium", 512, 256, 1024, 256, net.LAYER, True, True),
    ("layer reference norm", 64, 64, 128, 64, net.LAYER, True, False),
]


@pytest.mark.parametrize("name,S,H,F,O,norm,bias,affine", TRAIN_CASES)
def test_transformer_training_step(rt, name, S, H, F, O, norm, bias, affine):
    say(f"training {name}")
    p = make_params(S, H, F, O, 50, bias=bias, affine=affine, norm=norm)
    X = synth.normal((S, H), 5)
    dY = synth.normal((S, O), 6)
    lr = np.float32(1e-3)
    T = net.Transformer(rt, p, S, H, F, O, norm, net.ENCODER_TRAINING)
    Y = T.forward(rt.array(X)).numpy()
    ref, cache = ex.transformer_forward(p, X, norm)
    assert rel(Y, ref) <= TOL
    dXd = rt.empty((S, H))
    grads = T.backward(rt.array(dY), float(lr), dXd, want_grads=True)
    rdX, rg = ex.transformer_backward(p, cache, dY, norm)
    errs = {"dX": rel(dXd.numpy(), rdX)}
    for k in net.TP_SLOTS:
        if rg.get(k) is None or p.get(k) is None:
            continue
        g = grads[k].numpy()
        if k == "BK":
            # d(BK) = column sums of dK = sum_i Q_i * sum_j dS_ij = 0 exactly
            # (softmax is invariant to the per-row shift a key bias adds), so
            # only rounding noise remains: bound it against the value bias
            # gradient's scale instead of a relative error to zero.
            errs[k] = float(np.max(np.abs(g)) / np.max(np.abs(rg["BV"])))
        else:
            errs[k] = rel(g, rg[k])
        # SGD identity on the updated parameter, from the returned gradient.
        new = T.param(k)
        assert np.array_equal(new, p[k] - lr * g), f"SGD update of {k}"
    print("  " + " ".join(f"{k}={v:.1e}" for k, v in errs.items()))
    bad = {k: v for k, v in errs.items() if v > TOL}
    assert not bad, bad


@pytest.mark.parametrize("norm,bias,affine,score_bytes",
                         [(net.LAYER, True, True, None), (net.RMS, False, True, None),
                          (net.LAYER, True, False, 64 * 160 * 4)])
def test_training_step_without_gradients_updates_the_same(rt, norm, bias, affine, score_bytes):
    """A step that keeps no gradients (the bias sums then feed only the SGD
    step, the Q/K/V weight updates write no dW), and one that also returns
    no input gradient (the library then owns dXp), leave every parameter
    bit for bit where the step that returns the gradients leaves it,
    unchunked and chunked (64-row chunks of a 160-row sequence)."""
    S, H, F, O = 160, 64, 192, 48
    say(f"training without gradients norm={norm} bias={bias} chunked={score_bytes}")
    p = make_params(S, H, F, O, 70, bias=bias, affine=affine, norm=norm)
    X, dY = synth.normal((S, H), 71), synth.normal((S, O), 72)
    models = [net.Transformer(rt, p, S, H, F, O, norm, net.ENCODER_TRAINING) for _ in range(3)]
    dxs = []
    for (want, keep_dx), T in zip(((True, True), (False, True), (False, False)), models):
        if score_bytes:
            T.set_score_bytes(score_bytes)
        T.forward(rt.array(X))
        dx = rt.empty((S, H)) if keep_dx else None
        T.backward(rt.array(dY), 1e-3, dx, want_grads=want)
        if keep_dx:
            dxs.append(dx.numpy())
    assert np.array_equal(dxs[0], dxs[1])
    for k in net.TP_SLOTS:
        if p.get(k) is None:
            continue
        for T in models[1:]:
            assert np.array_equal(models[0].param(k), T.param(k)), k
    for T in models:
        T.close()


def test_transformer_training_c5_full_size(rt):
    """BASELINE config 5 at full size (S=4096, H=2048, F=8192, O=2048,
    LayerNorm with gamma/beta): one step against the f64 oracle, every one of
    the 17 parameter gradients and dX, and the SGD identity on every updated
    parameter."""
    S, H, F, O = 4096, 2048, 8192, 2048
    say("training C5 full size")
    p = make_params(S, H, F, O, 60, bias=True, affine=True, norm=net.LAYER)
    for k in ("BQ", "BK", "BV", "B1", "B2", "BO"):
        p[k] = np.zeros_like(p[k])
    X = synth.normal((S, H), 7)
    dY = synth.normal((S, O), 8)
    T = net.Transformer(rt, p, S, H, F, O, net.LAYER, net.ENCODER_TRAINING)
    Y = T.forward(rt.array(X)).numpy()
    dXd = rt.empty((S, H))
    grads = T.backward(rt.array(dY), 1e-3, dXd, want_grads=True)
    ref, cache = ex.transformer_forward(p, X, net.LAYER)
    errs = {"Y": rel(Y, ref)}
    rdX, rg = ex.transformer_backward(p, cache, dY, net.LAYER)
    errs["dX"] = rel(dXd.numpy(), rdX)
    lr = np.float32(1e-3)
    assert sorted(net.TP_SLOTS) == sorted(ex.SLOTS)
    for k in net.TP_SLOTS:  # all 17 parameter slots
        g = grads[k].numpy()
        if k == "BK":
            # identically zero in exact arithmetic (softmax shift invariance):
            # bounded against the value-bias gradient's scale.
            errs[k] = float(np.max(np.abs(g)) / np.max(np.abs(rg["BV"])))
        else:
            errs[k] = rel(g, rg[k])
        # SGD identity: the updated parameter is p - lr * g, bit for bit.
        assert np.array_equal(T.param(k), p[k] - lr * g), f"SGD update of {k}"
    print("  " + " ".join(f"{k}={v:.1e}" for k, v in errs.items()))
    bad = {k: v for k, v in errs.items() if v > TOL}
    assert not bad, bad


@pytest.mark.parametrize("act", [ex.IDENTITY, ex.RELU, ex.SILU])
@pytest.mark.parametrize("norm", [net.LAYER, net.RMS])
def test_transformer_ffn_activations(rt, act, norm):
    """The FFN's first layer with each activation the reference offers
    (linear.rs:21-70) besides GELU: encoder and decoder forward, and the
    training step's gradients and SGD identity, against the f64 oracle."""
    S, H, F, O = 64, 64, 192, 48
    say(f"ffn activation {act} norm {norm}")
    p = make_params(S, H, F, O, 60 + act, bias=True, affine=True, norm=norm)
    X = synth.normal((S, H), 7)
    for kind in (net.ENCODER_INFERENCE, net.DECODER_INFERENCE):
        T = net.Transformer(rt, p, S, H, F, O, norm, kind, ffn_activation=act)
        Y = T.forward(rt.array(X)).numpy()
        ref, _ = ex.transformer_forward(p, X, norm, act, causal=(kind == net.DECODER_INFERENCE))
        assert rel(Y, ref) <= TOL, kind
        T.close()
    dY = synth.normal((S, O), 8)
    lr = np.float32(1e-3)
    T = net.Transformer(rt, p, S, H, F, O, norm, net.ENCODER_TRAINING, ffn_activation=act)
    Y = T.forward(rt.array(X)).numpy()
    ref, cache = ex.transformer_forward(p, X, norm, act)
    assert rel(Y, ref) <= TOL
    dXd = rt.empty((S, H))
    grads = T.backward(rt.array(dY), float(lr), dXd, want_grads=True)
    rdX, rg = ex.transformer_backward(p, cache, dY, norm, act)
    assert rel(dXd.numpy(), rdX) <= TOL
    for k in net.TP_SLOTS:
        if rg.get(k) is None or p.get(k) is None or k == "BK":
            continue
        g = grads[k].numpy()
        assert rel(g, rg[k]) <= TOL, k
        assert np.array_equal(T.param(k), p[k] - lr * g), f"SGD update of {k}"
    T.close()
