"""Checkpoint round trips on the GPU, through the C ABI.

For every model family: a file written by the Python restatement of the
format (oracle/checkpoint.py) loads into a device model whose parameters are
bit-identical to the arrays written; a device model saves a .toml that tomli
parses to exactly the restatement's metadata for the same parameters and a
.bin byte-identical to the restatement's; a model loaded back from its own
save gives bit-identical outputs (and, for training kinds, bit-identical
parameters after one more SGD step) to the model that saved it.
"""
import os

import numpy as np
import pytest

from oracle import checkpoint as ck
from oxforge import _lib, net

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def rnd(shape, seed, scale=0.2):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def transformer_params(S, H, F, O, seed=0, bias=True, norm=net.LAYER, affine=True):
    p = {"WQ": rnd((H, H), seed), "WK": rnd((H, H), seed + 1), "WV": rnd((H, H), seed + 2),
         "POS": rnd((S, H), seed + 3), "W1": rnd((H, F), seed + 4), "W2": rnd((F, H), seed + 5),
         "WO": rnd((H, O), seed + 6)}
    for i, (k, n) in enumerate((("BQ", H), ("BK", H), ("BV", H), ("B1", F), ("B2", H),
                                ("BO", O))):
        p[k] = rnd((n,), seed + 10 + i) if bias else None
    for k in ("G1", "BE1", "G2", "BE2"):
        p[k] = None
    if affine:
        p["G1"] = 1 + rnd((H,), seed + 20)
        p["G2"] = 1 + rnd((H,), seed + 21)
        if norm == net.LAYER:
            p["BE1"], p["BE2"] = rnd((H,), seed + 22), rnd((H,), seed + 23)
    return p


def check_saved(path, expected_meta, expected_blocks):
    meta, data = ck.read(path)
    assert meta == expected_meta
    ck.validate(meta, os.path.getsize(path + ".bin"))
    raw = open(path + ".bin", "rb").read()
    assert raw == b"".join(np.ascontiguousarray(b, "<f4").tobytes() for b in expected_blocks)


# ------------------------------------------------------------------ Linear
@pytest.mark.parametrize("bias,act", [(True, 1), (False, 0), (True, 3)])
def test_linear_round_trip(rt, tmp_path, bias, act):
    say(f"checkpoint linear bias={bias} act={act}")
    W, b = rnd((40, 24), 1), (rnd((24,), 2) if bias else None)
    src = str(tmp_path / "oracle_lin")
    ck.write_linear(src, W, b, act)
    m = net.load(rt, src, net.CK_LINEAR)
    assert (m.n_in, m.n_out) == (40, 24)
    np.testing.assert_array_equal(m.param(0), W)
    if bias:
        np.testing.assert_array_equal(m.param(1), b)
    else:
        assert m.param(1) is None

    out = str(tmp_path / "saved_lin")
    m.save(out)
    cur, blocks = ck.Cursor(), []
    body = ck.linear_meta(W, b, act, cur, blocks)
    check_saved(out, ck.document("linear", body, "saved_lin.bin", cur.position), blocks)

    X = rt.array(rnd((33, 40), 3, 1.0))
    back = net.load(rt, out + ".toml", net.CK_LINEAR)
    np.testing.assert_array_equal(back.forward(X).numpy(), m.forward(X).numpy())
    for h in (m, back):
        h.close()


# --------------------------------------------------------------------- MLP
@pytest.mark.parametrize("training", [False, True])
def test_mlp_round_trip(rt, tmp_path, training):
    say(f"checkpoint mlp training={training}")
    dims = (32, 48, 48, 32)
    layers = [(rnd((dims[i], dims[i + 1]), 10 + i), rnd((dims[i + 1],), 20 + i) if i != 1
               else None, (1, 2, 0)[i]) for i in range(3)]
    src = str(tmp_path / "oracle_mlp")
    ck.write_mlp(src, layers, (0, 3))
    kind = net.CK_MLP_TRAINING if training else net.CK_MLP_INFERENCE
    m = net.load(rt, src, kind)
    assert m.dims == list(dims)
    for i, (W, b, _) in enumerate(layers):
        np.testing.assert_array_equal(m.param(i, 0), W)
        if b is not None:
            np.testing.assert_array_equal(m.param(i, 1), b)

    out = str(tmp_path / "saved_mlp")
    m.save(out)
    cur, blocks = ck.Cursor(), []
    body = ck.mlp_meta(layers, (0, 3), cur, blocks)
    check_saved(out, ck.document("mlp", body, "saved_mlp.bin", cur.position), blocks)

    back = net.load(rt, out, kind)
    X = rt.array(rnd((64, 32), 5, 1.0))
    np.testing.assert_array_equal(back.forward(X).numpy(), m.forward(X).numpy())
    if training:
        dY = rt.array(rnd((64, 32), 6))
        np.testing.assert_array_equal(back.backward(dY, 0.01).numpy(),
                                      m.backward(dY, 0.01).numpy())
        for i in range(3):
            np.testing.assert_array_equal(back.param(i, 0), m.param(i, 0))
    for h in (m, back):
        h.close()


# ------------------------------------------------------------- transformer
KINDS = {net.CK_ENCODER_INFERENCE: net.ENCODER_INFERENCE,
         net.CK_ENCODER_TRAINING: net.ENCODER_TRAINING,
         net.CK_DECODER_INFERENCE: net.DECODER_INFERENCE}


@pytest.mark.parametrize("ck_kind", list(KINDS))
@pytest.mark.parametrize("norm,affine,bias", [(net.LAYER, True, True), (net.RMS, True, False),
                                              (net.LAYER, False, True)])
def test_transformer_round_trip(rt, tmp_path, ck_kind, norm, affine, bias):
    say(f"checkpoint transformer kind={ck_kind} norm={norm} affine={affine} bias={bias}")
    S, H, F, O = 64, 64, 128, 32
    P = transformer_params(S, H, F, O, seed=ck_kind * 7, bias=bias, norm=norm, affine=affine)
    src = str(tmp_path / "oracle_tr")
    ck.write_transformer(src, P, norm, 1)
    m = net.load(rt, src, ck_kind)
    d = m.desc
    assert (d.seq, d.hidden, d.ffn, d.out) == (S, H, F, O)
    assert (d.norm_type, d.kind, d.ffn_activation) == (norm, KINDS[ck_kind], 1)
    for k in net.TP_SLOTS:
        got = m.param(k)
        if P[k] is None:
            assert got is None, k
        else:
            np.testing.assert_array_equal(got, P[k], err_msg=k)

    out = str(tmp_path / "saved_tr")
    m.save(out)
    cur, blocks = ck.Cursor(), []
    body = ck.transformer_meta(P, norm, 1, cur, blocks)
    check_saved(out, ck.document("transformer", body, "saved_tr.bin", cur.position), blocks)

    # The model built from the same parameters by the creation entry point
    # computes exactly what the loaded one does.
    made = net.Transformer(rt, P, S, H, F, O, norm_type=norm, kind=KINDS[ck_kind])
    back = net.load(rt, out, ck_kind)
    X = rt.array(rnd((S, H), 9, 1.0))
    ref = made.forward(X).numpy()
    np.testing.assert_array_equal(m.forward(X).numpy(), ref)
    np.testing.assert_array_equal(back.forward(X).numpy(), ref)
    if ck_kind == net.CK_ENCODER_TRAINING:
        dY = rt.array(rnd((S, O), 10))
        for h in (made, back):
            h.backward(dY, 0.01)
        for k in net.TP_SLOTS:
            a, b = made.param(k), back.param(k)
            assert (a is None) == (b is None), k
            if a is not None:
                np.testing.assert_array_equal(b, a, err_msg=k)
    for h in (m, made, back):
        h.close()


def test_trained_transformer_resumes(rt, tmp_path):
    """Train, save, load, train on: identical to training without the stop."""
    say("checkpoint transformer resume")
    S, H, F, O = 32, 64, 96, 64
    P = transformer_params(S, H, F, O, seed=3)
    a = net.Transformer(rt, P, S, H, F, O, kind=net.ENCODER_TRAINING)
    X = rt.array(rnd((S, H), 11, 1.0))
    dY = rt.array(rnd((S, O), 12))
    a.forward(X)
    a.backward(dY, 0.05)
    path = str(tmp_path / "resume")
    a.save(path)
    b = net.load(rt, path, net.CK_ENCODER_TRAINING)
    for h in (a, b):
        h.forward(X)
        h.backward(dY, 0.05)
    np.testing.assert_array_equal(b.forward(X).numpy(), a.forward(X).numpy())
    for h in (a, b):
        h.close()


def test_load_errors(rt, tmp_path):
    say("checkpoint load errors")
    P = transformer_params(8, 16, 32, 8)
    path = str(tmp_path / "tr")
    ck.write_transformer(path, P, net.LAYER, 1)
    # A transformer file is not a Linear or an MLP (model type check).
    for kind in (net.CK_LINEAR, net.CK_MLP_INFERENCE):
        with pytest.raises(_lib.ForgeError) as e:
            net.load(rt, path, kind)
        assert e.value.status == _lib.FORGE_EINVAL and "model type" in str(e.value)
    # A three-layer feed-forward network loads through the C++ API only.
    cur, blocks = ck.Cursor(), []
    g = P.get
    body = {"block_count": 1, "attention_residual": True, "feed_forward_residual": True,
            "normalization": "layer"}
    q = ck.linear_meta(P["WQ"], g("BQ"), 0, cur, blocks)
    k = ck.linear_meta(P["WK"], g("BK"), 0, cur, blocks)
    v = ck.linear_meta(P["WV"], g("BV"), 0, cur, blocks)
    body["position"] = cur.matrix(8, 16)
    blocks.append(P["POS"])
    body.update(query=q, key=k, value=v)
    body["feed_forward"] = ck.mlp_meta([(P["W1"], None, 1), (rnd((32, 32), 1), None, 1),
                                        (P["W2"], None, 0)], None, cur, blocks)
    body["output"] = ck.linear_meta(P["WO"], None, 0, cur, blocks)
    ck.write(path, "transformer", body, blocks, cur.position)
    assert net.inspect(path) == ("transformer", cur.position)
    with pytest.raises(_lib.ForgeError) as e:
        net.load(rt, path, net.CK_ENCODER_INFERENCE)
    assert "two-layer" in str(e.value)
    with pytest.raises(ValueError):
        net.load(rt, path, 17)
