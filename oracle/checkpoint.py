"""Restatement of the reference's checkpoint format version 1 in Python.

TEST INFRASTRUCTURE ONLY: it writes checkpoints from numpy parameters and
reads them back, as the independent side of the checkpoint parity tests (the
product's reader and writer are C++ and never import this).  Metadata is
built as nested dicts in the field order of the reference's serde structs and
emitted as TOML the way a pretty TOML serializer lays such a document out;
the tests parse every file, ours and the product's, with tomli (an
independent TOML parser).  Reference files (src/net/):

  checkpoint/model.rs:23-51   file structs (format_version, model_type,
                              scalar_type, data_file, data_bytes, <model>)
  metadata.rs:5-18, 36-52     MatrixMetadata / VectorMetadata, cursor
  linear.rs:79-114            LinearMetadata, parameter order weights, bias
  mlp.rs:21-34, 99-119        MlpMetadata (residual omitted when absent)
  transformer/inference.rs:12-24, 52-73
                              TransformerMetadata; parameter order Q, K, V,
                              position, feed-forward layers, output
  checkpoint/io.rs:66-177     .bin = parameters as contiguous f32 LE
  checkpoint/model.rs:350-543 validation (restated in validate())

The gamma/beta extension tables (norm1_gamma, norm1_beta, norm2_gamma,
norm2_beta, after the output projection) are this build's, not the
reference's.
"""
from __future__ import annotations

import os

import numpy as np

ACTIVATIONS = ["identity", "gelu", "relu", "silu"]
NORMS = ["rms", "layer"]


class Cursor:
    """MetadataCursor (metadata.rs:36-52): byte ranges in parameter order."""

    def __init__(self):
        self.position = 0

    def matrix(self, rows, cols):
        start = self.position
        self.position += rows * cols * 4
        return {"rows": rows, "cols": cols, "byte_start": start, "byte_end": self.position}

    def vector(self, n):
        start = self.position
        self.position += n * 4
        return {"len": n, "byte_start": start, "byte_end": self.position}


def linear_meta(W, b, activation, cur, blocks):
    """Linear::get_meta_data / get_data (linear.rs:97-114)."""
    m = {"input_neurons": W.shape[0], "output_neurons": W.shape[1],
         "activation": ACTIVATIONS[activation], "weights": cur.matrix(*W.shape)}
    blocks.append(W)
    if b is not None:
        m["bias"] = cur.vector(b.shape[0])
        blocks.append(b)
    return m


def mlp_meta(layers, res_range, cur, blocks):
    """MlpExecutor::get_meta_data / get_data (mlp.rs:99-119).
    layers: [(W, b or None, activation), ...]"""
    m = {"layer_count": len(layers), "loss": "mean_squared_error"}
    if res_range is not None:
        m["residual"] = {"start": res_range[0], "end": res_range[1]}
    m["layers"] = [linear_meta(W, b, a, cur, blocks) for W, b, a in layers]
    return m


def transformer_meta(p, norm_type, ffn_activation, cur, blocks):
    """InferenceBlock::get_meta_data / get_data (inference.rs:52-73) for the
    single-head block with a two-layer feed-forward network; p holds WQ, BQ,
    WK, BK, WV, BV, POS, W1, B1, W2, B2, WO, BO and optionally G1, BE1, G2,
    BE2 (None or absent = no such parameter)."""
    g = p.get
    q = linear_meta(p["WQ"], g("BQ"), 0, cur, blocks)
    k = linear_meta(p["WK"], g("BK"), 0, cur, blocks)
    v = linear_meta(p["WV"], g("BV"), 0, cur, blocks)
    pos = cur.matrix(*p["POS"].shape)
    blocks.append(p["POS"])
    ffn = mlp_meta([(p["W1"], g("B1"), ffn_activation), (p["W2"], g("B2"), 0)], None, cur, blocks)
    out = linear_meta(p["WO"], g("BO"), 0, cur, blocks)
    m = {"block_count": 1, "attention_residual": True, "feed_forward_residual": True,
         "normalization": NORMS[norm_type], "position": pos, "query": q, "key": k, "value": v,
         "feed_forward": ffn, "output": out}
    for key, slot in (("norm1_gamma", "G1"), ("norm1_beta", "BE1"), ("norm2_gamma", "G2"),
                      ("norm2_beta", "BE2")):
        if g(slot) is not None:
            m[key] = cur.vector(p[slot].shape[0])
            blocks.append(p[slot])
    return m


def document(model_type, body, data_file, data_bytes):
    """The file struct of model.rs:23-51."""
    return {"format_version": 1, "model_type": model_type, "scalar_type": "f32_le",
            "data_file": data_file, "data_bytes": data_bytes, model_type: body}


def _scalar(v):
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, (int, np.integer)):
        return str(int(v))
    if isinstance(v, str):
        return '"' + v.replace("\\", "\\\\").replace('"', '\\"') + '"'
    raise TypeError(type(v))


def to_toml(doc, prefix=""):
    """TOML text of a nested dict: plain keys first, then each sub-table under
    a [dotted.header] and each list of dicts as [[dotted.header]] entries,
    in insertion order."""
    lines = []
    for k, v in doc.items():
        if not isinstance(v, (dict, list)):
            lines.append(f"{k} = {_scalar(v)}")
    for k, v in doc.items():
        path = f"{prefix}{k}"
        if isinstance(v, dict):
            lines.append(f"\n[{path}]")
            lines.append(to_toml(v, path + ".").rstrip("\n"))
        elif isinstance(v, list):
            for item in v:
                lines.append(f"\n[[{path}]]")
                lines.append(to_toml(item, path + ".").rstrip("\n"))
    return "\n".join(x for x in lines if x != "") + "\n"


def write(path, model_type, body, blocks, data_bytes):
    """Writes <path>.toml and <path>.bin (path without extension)."""
    data_file = os.path.basename(path) + ".bin"
    with open(path + ".toml", "w") as f:
        f.write(to_toml(document(model_type, body, data_file, data_bytes)))
    data = b"".join(np.ascontiguousarray(b, dtype="<f4").tobytes() for b in blocks)
    assert len(data) == data_bytes
    with open(path + ".bin", "wb") as f:
        f.write(data)


def write_linear(path, W, b=None, activation=0):
    cur, blocks = Cursor(), []
    body = linear_meta(W, b, activation, cur, blocks)
    write(path, "linear", body, blocks, cur.position)


def write_mlp(path, layers, res_range=None):
    cur, blocks = Cursor(), []
    body = mlp_meta(layers, res_range, cur, blocks)
    write(path, "mlp", body, blocks, cur.position)


def write_transformer(path, params, norm_type, ffn_activation):
    cur, blocks = Cursor(), []
    body = transformer_meta(params, norm_type, ffn_activation, cur, blocks)
    write(path, "transformer", body, blocks, cur.position)


def read(path):
    """(metadata dict, .bin as a float32 array) of <path>.toml."""
    import tomli

    with open(path + ".toml", "rb") as f:
        meta = tomli.load(f)
    data = np.fromfile(os.path.join(os.path.dirname(path), meta["data_file"]), dtype="<f4")
    return meta, data


def tensor(data, m):
    """The parameter that a Matrix/VectorMetadata range describes."""
    a = data[m["byte_start"] // 4: m["byte_end"] // 4]
    return a.reshape(m["rows"], m["cols"]) if "rows" in m else a


class Invalid(ValueError):
    pass


def validate(meta, file_bytes):
    """model.rs:350-543 and io.rs:125-140: header, contiguous ranges from 0
    to data_bytes, shapes and connectivity, data-file size."""
    if meta.get("format_version") != 1:
        raise Invalid("unsupported checkpoint format version")
    mtype = meta.get("model_type")
    if mtype not in ("linear", "mlp", "transformer") or mtype not in meta:
        raise Invalid("model type")
    if meta.get("scalar_type") != "f32_le":
        raise Invalid("unsupported scalar encoding")
    data_file = meta["data_file"]
    if data_file in ("", ".", "..") or "/" in data_file:
        raise Invalid("checkpoint data_file must be a plain file name")
    pos = [0]

    def rng(m, n):
        if m["byte_start"] != pos[0] or m["byte_end"] != pos[0] + 4 * n:
            raise Invalid("is not the expected contiguous range")
        pos[0] += 4 * n

    def lin(m):
        if m["activation"] not in ACTIVATIONS:
            raise Invalid("unknown activation")
        if m["input_neurons"] == 0 or m["output_neurons"] == 0:
            raise Invalid("Linear dimensions must be non-zero")
        w = m["weights"]
        if (w["rows"], w["cols"]) != (m["input_neurons"], m["output_neurons"]):
            raise Invalid("Linear weight shape does not match its neuron counts")
        rng(w, w["rows"] * w["cols"])
        if "bias" in m:
            if m["bias"]["len"] != m["output_neurons"]:
                raise Invalid("Linear bias length does not match output neurons")
            rng(m["bias"], m["bias"]["len"])

    def mlp(m):
        layers = m.get("layers", [])
        if m["loss"] != "mean_squared_error":
            raise Invalid("unknown loss")
        if m["layer_count"] == 0 or m["layer_count"] != len(layers):
            raise Invalid("layer_count")
        for i, layer in enumerate(layers):
            lin(layer)
            if i > 0 and layers[i - 1]["output_neurons"] != layer["input_neurons"]:
                raise Invalid("expects")
        if "residual" in m:
            s, e = m["residual"]["start"], m["residual"]["end"]
            if s >= e or e > len(layers):
                raise Invalid("invalid MLP residual range")
            if layers[s]["input_neurons"] != layers[e - 1]["output_neurons"]:
                raise Invalid("residual connects")

    body = meta[mtype]
    if mtype == "linear":
        lin(body)
    elif mtype == "mlp":
        mlp(body)
    else:
        if body["normalization"] not in NORMS:
            raise Invalid("unknown normalization")
        if body["block_count"] != 1:
            raise Invalid("exactly one block")
        if not (body["attention_residual"] and body["feed_forward_residual"]):
            raise Invalid("both residual paths")
        for key in ("query", "key", "value"):
            lin(body[key])
        p = body["position"]
        rng(p, p["rows"] * p["cols"])
        mlp(body["feed_forward"])
        lin(body["output"])
        emb = p["cols"]
        if p["rows"] == 0 or emb == 0:
            raise Invalid("position matrix dimensions must be non-zero")
        if any(body[k]["input_neurons"] != emb for k in ("query", "key", "value")):
            raise Invalid("Q/K/V input dimensions")
        if body["query"]["output_neurons"] != body["key"]["output_neurons"]:
            raise Invalid("query and key dimensions must match")
        if body["value"]["output_neurons"] != emb:
            raise Invalid("value output dimension")
        ff = body["feed_forward"]["layers"]
        if ff[0]["input_neurons"] != emb or ff[-1]["output_neurons"] != emb:
            raise Invalid("feed-forward input/output")
        if body["output"]["input_neurons"] != emb:
            raise Invalid("output projection input")
        for key in ("norm1_gamma", "norm1_beta", "norm2_gamma", "norm2_beta"):
            if key in body:
                if body[key]["len"] != emb:
                    raise Invalid("norm gamma/beta length")
                if key.endswith("beta") and body["normalization"] != "layer":
                    raise Invalid("norm beta is only defined for LayerNorm")
                rng(body[key], body[key]["len"])
    if pos[0] != meta["data_bytes"]:
        raise Invalid("parameter ranges end at")
    if file_bytes != meta["data_bytes"]:
        raise Invalid("data file has")
