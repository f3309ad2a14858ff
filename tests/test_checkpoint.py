"""Checkpoint format version 1 without a GPU: the C++ reader's validation
(through forge_checkpoint_inspect, which parses and checks a checkpoint
without touching a device) against files written by the Python restatement
of the format (oracle/checkpoint.py), and that restatement against an
independent TOML parser (tomli).

Every rejection case is checked twice, with the same expected outcome: the
product (C++) and the restatement of model.rs:350-543 must both refuse it.
The reference holds no checkpoint fixtures; the cases are built so that each
breaks exactly one rule of the format (a shifted range, a wrong count, a
path component, ...), so a validator that skips that rule accepts the file.
"""
import copy
import os

import numpy as np
import pytest
import tomli

from oracle import checkpoint as ck
from oxforge import _lib, net


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def transformer_params(S=8, H=16, F=32, O=12, seed=0, bias=True, norm=net.LAYER, affine=True):
    p = {"WQ": rnd((H, H), seed), "WK": rnd((H, H), seed + 1), "WV": rnd((H, H), seed + 2),
         "POS": rnd((S, H), seed + 3), "W1": rnd((H, F), seed + 4), "W2": rnd((F, H), seed + 5),
         "WO": rnd((H, O), seed + 6)}
    for i, (k, n) in enumerate((("BQ", H), ("BK", H), ("BV", H), ("B1", F), ("B2", H),
                                ("BO", O))):
        p[k] = rnd((n,), seed + 10 + i) if bias else None
    if affine:
        p["G1"], p["G2"] = rnd((H,), 20), rnd((H,), 21)
        if norm == net.LAYER:
            p["BE1"], p["BE2"] = rnd((H,), 22), rnd((H,), 23)
    return p


def mlp_layers(dims=(6, 10, 10, 6), seed=0, bias=(True, False, True), acts=(1, 2, 0)):
    return [(rnd((dims[i], dims[i + 1]), seed + i), rnd((dims[i + 1],), seed + 9 + i)
             if bias[i] else None, acts[i]) for i in range(len(dims) - 1)]


def cases(tmp_path):
    """(path without extension, model_type) for each model family."""
    out = []
    p = str(tmp_path / "lin_bias")
    ck.write_linear(p, rnd((7, 5), 1), rnd((5,), 2), 1)
    out.append((p, "linear"))
    p = str(tmp_path / "lin_plain")
    ck.write_linear(p, rnd((3, 9), 3))
    out.append((p, "linear"))
    p = str(tmp_path / "mlp_res")
    ck.write_mlp(p, mlp_layers(), (0, 3))
    out.append((p, "mlp"))
    p = str(tmp_path / "mlp_plain")
    ck.write_mlp(p, mlp_layers((4, 8), bias=(True,), acts=(3,)))
    out.append((p, "mlp"))
    p = str(tmp_path / "tr_layer")
    ck.write_transformer(p, transformer_params(), net.LAYER, 1)
    out.append((p, "transformer"))
    p = str(tmp_path / "tr_rms_plain")
    ck.write_transformer(p, transformer_params(bias=False, norm=net.RMS, affine=False), net.RMS, 3)
    out.append((p, "transformer"))
    return out


def status_of(fn):
    with pytest.raises(_lib.ForgeError) as e:
        fn()
    return e.value.status, str(e.value)


# ------------------------------------------------- the restatement itself
def test_writer_emits_the_document_tomli_reads(tmp_path):
    for path, mtype in cases(tmp_path):
        with open(path + ".toml", "rb") as f:
            meta = tomli.load(f)
        assert meta["format_version"] == 1 and meta["model_type"] == mtype
        assert meta["scalar_type"] == "f32_le"
        assert meta["data_file"] == os.path.basename(path) + ".bin"
        assert meta["data_bytes"] == os.path.getsize(path + ".bin")
        ck.validate(meta, os.path.getsize(path + ".bin"))


def test_parameter_layout_is_contiguous_f32_le(tmp_path):
    """Each range of the metadata holds exactly the parameter it names."""
    W, b = rnd((7, 5), 1), rnd((5,), 2)
    p = str(tmp_path / "x")
    ck.write_linear(p, W, b, 2)
    meta, data = ck.read(p)
    lin = meta["linear"]
    assert lin["weights"] == {"rows": 7, "cols": 5, "byte_start": 0, "byte_end": 140}
    assert lin["bias"] == {"len": 5, "byte_start": 140, "byte_end": 160}
    assert lin["activation"] == "relu"
    raw = open(p + ".bin", "rb").read()
    assert raw[:4] == W[0, 0].astype("<f4").tobytes()
    np.testing.assert_array_equal(ck.tensor(data, lin["weights"]), W)
    np.testing.assert_array_equal(ck.tensor(data, lin["bias"]), b)


def test_transformer_parameter_order(tmp_path):
    """Q, K, V (weights then bias), position, FFN layers, output, then the
    gamma/beta extension (inference.rs:52-73)."""
    P = transformer_params()
    p = str(tmp_path / "t")
    ck.write_transformer(p, P, net.LAYER, 1)
    meta, data = ck.read(p)
    t = meta["transformer"]
    order = [t["query"]["weights"], t["query"]["bias"], t["key"]["weights"], t["key"]["bias"],
             t["value"]["weights"], t["value"]["bias"], t["position"],
             t["feed_forward"]["layers"][0]["weights"], t["feed_forward"]["layers"][0]["bias"],
             t["feed_forward"]["layers"][1]["weights"], t["feed_forward"]["layers"][1]["bias"],
             t["output"]["weights"], t["output"]["bias"], t["norm1_gamma"], t["norm1_beta"],
             t["norm2_gamma"], t["norm2_beta"]]
    names = ["WQ", "BQ", "WK", "BK", "WV", "BV", "POS", "W1", "B1", "W2", "B2", "WO", "BO",
             "G1", "BE1", "G2", "BE2"]
    assert [m["byte_start"] for m in order] == sorted(m["byte_start"] for m in order)
    for m, n in zip(order, names):
        np.testing.assert_array_equal(ck.tensor(data, m), P[n])
    assert t["feed_forward"]["layers"][0]["activation"] == "gelu"
    assert t["normalization"] == "layer" and t["block_count"] == 1


# ------------------------------------------------------- the C++ reader
def test_inspect_accepts_every_family(tmp_path):
    for path, mtype in cases(tmp_path):
        size = os.path.getsize(path + ".bin")
        assert net.inspect(path) == (mtype, size)
        assert net.inspect(path + ".toml") == (mtype, size)


def rewrite(path, meta):
    with open(path + ".toml", "w") as f:
        f.write(ck.to_toml(meta))


def mutations():
    """(name, model family index in cases(), mutate(meta, path), message part)."""

    def setk(keys, value):
        def f(meta, path):
            d = meta
            for k in keys[:-1]:
                d = d[k]
            d[keys[-1]] = value
        return f

    def shift(keys):
        def f(meta, path):
            d = meta
            for k in keys:
                d = d[k]
            d["byte_start"] += 4
            d["byte_end"] += 4
        return f

    def drop(keys):
        def f(meta, path):
            d = meta
            for k in keys[:-1]:
                d = d[k]
            del d[keys[-1]]
        return f

    def truncate(meta, path):
        with open(path + ".bin", "r+b") as f:
            f.truncate(os.path.getsize(path + ".bin") - 4)

    def swap_qk(meta, path):
        t = meta["transformer"]
        t["query"], t["key"] = t["key"], t["query"]

    def add_layer_count(meta, path):
        meta["mlp"]["layer_count"] += 1

    def break_connectivity(meta, path):
        # A consistent layer 1 of the wrong width, ranges laid out again so
        # that only the connectivity rule is broken.
        layers = meta["mlp"]["layers"]
        layers[1]["input_neurons"] += 1
        layers[1]["weights"]["rows"] += 1
        cur = ck.Cursor()
        for layer in layers:
            layer["weights"] = cur.matrix(layer["weights"]["rows"], layer["weights"]["cols"])
            if "bias" in layer:
                layer["bias"] = cur.vector(layer["bias"]["len"])
        meta["data_bytes"] = cur.position

    return [
        ("version", 0, setk(["format_version"], 2), "format version"),
        ("model type", 0, setk(["model_type"], "mlp"), "mlp"),
        ("scalar", 0, setk(["scalar_type"], "f64_le"), "scalar encoding"),
        ("shifted weights", 0, shift(["linear", "weights"]), "contiguous range"),
        ("shifted bias", 0, shift(["linear", "bias"]), "contiguous range"),
        ("data bytes", 0, setk(["data_bytes"], 156), "parameter ranges end at"),
        ("truncated bin", 0, truncate, "data file has"),
        ("weight shape", 0, setk(["linear", "weights", "rows"], 6), "weight shape"),
        ("bias length", 0, setk(["linear", "bias", "len"], 4), "bias length"),
        ("zero dims", 1, setk(["linear", "input_neurons"], 0), "non-zero"),
        ("path data_file", 0, setk(["data_file"], "../lin_bias.bin"), "plain file name"),
        ("dir data_file", 0, setk(["data_file"], "sub/lin_bias.bin"), "plain file name"),
        ("layer count", 2, add_layer_count, "layer_count"),
        ("connectivity", 2, break_connectivity, "expects"),
        ("residual range", 2, setk(["mlp", "residual", "end"], 4), "residual range"),
        ("residual empty", 2, setk(["mlp", "residual", "start"], 3), "residual range"),
        ("residual dims", 2, setk(["mlp", "residual"], {"start": 0, "end": 1}),
         "residual connects"),
        ("unknown activation", 0, setk(["linear", "activation"], "tanh"), "activation"),
        ("block count", 4, setk(["transformer", "block_count"], 2), "one block"),
        ("attention residual", 4, setk(["transformer", "attention_residual"], False),
         "residual paths"),
        ("swapped q/k order", 4, swap_qk, "contiguous range"),
        ("position order", 4, shift(["transformer", "position"]), "contiguous range"),
        ("norm extension len", 4, setk(["transformer", "norm2_beta", "len"], 15),
         "norm gamma/beta length"),
        ("beta with rms", 4, setk(["transformer", "normalization"], "rms"), "LayerNorm"),
        ("unknown norm", 5, setk(["transformer", "normalization"], "batch"), "normalization"),
        ("missing output", 5, drop(["transformer", "output"]), "output"),
    ]


@pytest.mark.parametrize("name,family,mutate,part", mutations(),
                         ids=[m[0] for m in mutations()])
def test_inspect_rejects(tmp_path, name, family, mutate, part):
    path, _ = cases(tmp_path)[family]
    with open(path + ".toml", "rb") as f:
        meta = tomli.load(f)
    meta = copy.deepcopy(meta)
    mutate(meta, path)
    rewrite(path, meta)
    with pytest.raises((ck.Invalid, KeyError)):
        ck.validate(meta, os.path.getsize(path + ".bin"))
    status, msg = status_of(lambda: net.inspect(path))
    assert status == _lib.FORGE_EINVAL, msg
    assert part in msg, msg


def test_paths(tmp_path):
    path, _ = cases(tmp_path)[0]
    # io.rs:20-29: another extension than .toml is refused before any I/O.
    status, msg = status_of(lambda: net.inspect(path + ".json"))
    assert status == _lib.FORGE_EINVAL and "must use .toml, not .json" in msg
    status, msg = status_of(lambda: net.inspect(str(tmp_path / "missing")))
    assert status == _lib.FORGE_EIO and "missing.toml" in msg
    os.remove(path + ".bin")
    status, msg = status_of(lambda: net.inspect(path))
    assert status == _lib.FORGE_EIO and "lin_bias.bin" in msg


def test_toml_syntax_accepted(tmp_path):
    """Equivalent spellings of the same document: comments, inline tables,
    dotted keys, literal strings, table order, underscores in integers."""
    path, _ = cases(tmp_path)[0]
    text = (
        "# a linear checkpoint\n"
        "format_version = 1 # trailing comment\n"
        "model_type = 'linear'\n"
        "scalar_type = \"f32_le\"\n"
        "data_file = \"lin_bias.bin\"\n"
        "data_bytes = 1_6_0\n"
        "[linear.bias]\n"
        "len = 5\n"
        "byte_start = 140\n"
        "byte_end = 160\n"
        "[linear]\n"
        "input_neurons = 7\n"
        "output_neurons = 5\n"
        "activation = \"gelu\"\n"
        "weights = { rows = 7, cols = 5, byte_start = 0, byte_end = 140 }\n")
    with open(path + ".toml", "w") as f:
        f.write(text)
    assert tomli.loads(text)["linear"]["weights"]["byte_end"] == 140
    assert net.inspect(path) == ("linear", 160)
    dotted = text.replace("weights = { rows = 7, cols = 5, byte_start = 0, byte_end = 140 }\n",
                          "weights.rows = 7\nweights.cols = 5\nweights.byte_start = 0\n"
                          "weights.byte_end = 140\n")
    with open(path + ".toml", "w") as f:
        f.write(dotted)
    assert net.inspect(path) == ("linear", 160)


@pytest.mark.parametrize("bad,part", [
    ("data_bytes = 160.0", "floating-point"),
    ("data_bytes = 160\ndata_bytes = 160", "duplicate key"),
    ("data_bytes = \"160", "unterminated string"),
    ("data_bytes = -160", "non-negative"),
    ("[linear", "bad table header"),
    ("data_bytes = 99999999999999999999999", "integer overflow"),
    ("data_bytes = 0160", "leading zeros"),
    ("data_bytes = 1__60", "underscore"),
    ("data_bytes = 160_", "underscore"),
    ("data_bytes = _160", "underscore"),
])
def test_toml_syntax_rejected(tmp_path, bad, part):
    path, _ = cases(tmp_path)[0]
    text = open(path + ".toml").read().replace("data_bytes = 160", bad)
    with open(path + ".toml", "w") as f:
        f.write(text)
    status, msg = status_of(lambda: net.inspect(path))
    assert status == _lib.FORGE_EINVAL and part in msg, msg


@pytest.mark.parametrize("tail,part", [
    ("[linear]\n", "defined twice"),
    ("[linear.weights]\n", "defined twice"),
])
def test_toml_table_defined_twice_rejected(tmp_path, tail, part):
    """A second [header] for a table, or a header for a table that dotted keys
    or an inline table already defined, is refused (TOML 1.0; tomli, an
    independent parser, refuses the same documents)."""
    path, _ = cases(tmp_path)[0]
    text = open(path + ".toml").read() + tail
    with pytest.raises(tomli.TOMLDecodeError):
        tomli.loads(text)
    with open(path + ".toml", "w") as f:
        f.write(text)
    status, msg = status_of(lambda: net.inspect(path))
    assert status == _lib.FORGE_EINVAL and part in msg, msg


def test_toml_header_after_dotted_keys_rejected(tmp_path):
    """linear.weights defined by dotted keys inside [linear], then given its
    own header: refused, as tomli refuses it."""
    path, _ = cases(tmp_path)[0]
    text = open(path + ".toml").read()
    text = text.replace("[linear.weights]\nrows = 7\ncols = 5\nbyte_start = 0\nbyte_end = 140\n",
                        "")
    text = text.replace('activation = "gelu"\n',
                        'activation = "gelu"\nweights.rows = 7\nweights.cols = 5\n'
                        'weights.byte_start = 0\nweights.byte_end = 140\n')
    assert tomli.loads(text)["linear"]["weights"]["byte_end"] == 140
    with open(path + ".toml", "w") as f:
        f.write(text)
    assert net.inspect(path) == ("linear", 160)
    bad = text + "[linear.weights]\n"
    with pytest.raises(tomli.TOMLDecodeError):
        tomli.loads(bad)
    with open(path + ".toml", "w") as f:
        f.write(bad)
    status, msg = status_of(lambda: net.inspect(path))
    assert status == _lib.FORGE_EINVAL and "defined twice" in msg, msg


def test_inspect_survives_mutated_files(tmp_path):
    """Fixed-seed mutations of valid files (byte flips, TOML punctuation and
    escapes inserted, cuts, duplicated spans, long runs, a short or long data
    file): the reader returns FORGE_OK, FORGE_EINVAL or FORGE_EIO for every
    one and never crashes.  (A longer run of the same mutations against an
    AddressSanitizer build of the host library found no memory errors.)"""
    import random

    bases = [p for p, _ in cases(tmp_path)]
    texts = {b: open(b + ".toml", "rb").read() for b in bases}
    special = [b'"', b"'", b"[", b"]]", b"=", b"\\", b"\n", b"#", b".", b"{", b"}", b",", b"_",
               b'"""', b"'''", b"\\U0010FFFF", b"9" * 40, b"\x00", b"\xff", b"\r\n",
               b"a.b.c.d = 1\n", b"{a={b={c=1}}}"]
    rng = random.Random(7)
    fz = str(tmp_path / "fz")
    seen = set()
    for _ in range(400):
        b = rng.choice(bases)
        t = bytearray(texts[b])
        for _ in range(rng.randint(1, 5)):
            op, pos = rng.randrange(5), rng.randrange(len(t) + 1)
            if op == 0 and t:
                t[rng.randrange(len(t))] = rng.randrange(256)
            elif op == 1:
                t[pos:pos] = rng.choice(special)
            elif op == 2:
                del t[pos:pos + rng.randint(1, 20)]
            elif op == 3:
                t = t[:pos]
            else:
                t[pos:pos] = b"x" * rng.choice([1, 256, 70000])
        name = os.path.basename(b).encode() + b".bin"
        with open(fz + ".toml", "wb") as f:
            f.write(bytes(t).replace(name, b"fz.bin"))
        data = open(b + ".bin", "rb").read()
        cut = rng.choice([None, None, 0, len(data) // 2, len(data) + 4])
        with open(fz + ".bin", "wb") as f:
            f.write(data if cut is None else data[:cut] if cut <= len(data) else data + bytes(4))
        try:
            net.inspect(fz)
            status = 0
        except _lib.ForgeError as e:
            status = e.status
        assert status in (0, 1, 6), status
        seen.add(status)
    assert seen >= {1}
