"""The C++ drop-in API (include/oxforge_net.hpp: CudaRuntime, Matrix, Vector,
streams, the buffer pool, conversions, Linear, MLP) exercised on the GPU by
the in-tree program oxide-forge_amd/lib/oxforge_cpp_api_test, built from
oxide-forge_amd/csrc/tests/cpp_api_test.cpp by the same Makefile as the
library.  Its checks compare against host arithmetic: bit-exact for copies,
fills, conversions and single rounded elementwise ops, 1e-4 relative for the
GEMM, 1e-5 absolute for softmax and the norms."""
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oxide-forge_amd", "lib", "oxforge_cpp_api_test")


def test_cpp_api_program_is_built():
    assert os.path.exists(BIN), "run __graft_entry__.build() (make -C oxide-forge_amd/csrc)"


@pytest.mark.gpu
def test_cpp_api_on_gpu(tmp_path):
    """Runs the program; its span group (DeviceSpan / DeviceSpanMut /
    VectorView / Matrix::row_views, span.rs:82-299, vector_view.rs:6-47,
    convert.rs:8-13) also writes its inputs and results, which are checked
    here against the oracle: VectorView::softmax of each row against the
    oracle's row softmax (1e-5 absolute) and map_sum of six functors
    against the f64 sum of the oracle's per-element map (1e-5 relative to
    the sum of magnitudes)."""
    from oracle import oracle as orc

    print("[case] C++ API program", flush=True)
    res = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True, timeout=100)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "FAIL" not in res.stdout
    rows, cols = 6, 1000
    x = np.fromfile(tmp_path / "spans_input.f32", np.float32).reshape(rows, cols)
    sm = np.fromfile(tmp_path / "spans_softmax.f32", np.float32).reshape(rows, cols)
    sums = np.fromfile(tmp_path / "spans_map_sum.f32", np.float32).reshape(rows, 6)
    assert np.max(np.abs(sm - orc.softmax_rows(x))) <= 1e-5
    fns = [(orc.MAP_IDENTITY, 0.0), (orc.MAP_SCALE, 0.5), (orc.MAP_ADD, 1.25),
           (orc.MAP_HALF_SQ, 0.0), (orc.MAP_EXP_SHIFT, 0.3), (orc.MAP_GELU, 0.0)]
    for r in range(rows):
        for k, (op, p0) in enumerate(fns):
            mapped = orc.map_(x[r], op, p0).astype(np.float64)
            ref = mapped.sum()
            tol = 1e-5 * max(1.0, np.abs(mapped).sum())
            assert abs(float(sums[r, k]) - ref) <= tol, (r, op, float(sums[r, k]), ref)


def _oracle_models(rng_seed=7):
    """Parameters of the five checkpoints the metadata test loads, and the
    oracle's metadata body and parameter blocks for each (oracle/checkpoint.py,
    the restatement of linear.rs:97-114, mlp.rs:99-119, inference.rs:52-73)."""
    from oracle import checkpoint as ock
    from oxforge import synth

    models = {}
    cur, blocks = ock.Cursor(), []
    W, b = synth.uniform((24, 40), rng_seed), synth.uniform((40,), rng_seed + 1)
    models["linear"] = ("linear", (W, b, 1), ock.linear_meta(W, b, 1, cur, blocks), blocks,
                        cur.position)
    cur, blocks = ock.Cursor(), []
    models["linear_nobias"] = ("linear", (W, None, 3), ock.linear_meta(W, None, 3, cur, blocks),
                               blocks, cur.position)
    layers = [(synth.uniform((16, 32), 20), synth.uniform((32,), 21), 1),
              (synth.uniform((32, 32), 22), None, 2),
              (synth.uniform((32, 16), 23), synth.uniform((16,), 24), 0)]
    cur, blocks = ock.Cursor(), []
    models["mlp"] = ("mlp", (layers, (0, 3)), ock.mlp_meta(layers, (0, 3), cur, blocks), blocks,
                     cur.position)
    S, H, F, O = 8, 16, 32, 12
    p = {"WQ": synth.xavier(H, H, 40), "BQ": synth.normal((H,), 41, 0.0, 0.1),
         "WK": synth.xavier(H, H, 42), "BK": None, "WV": synth.xavier(H, H, 43),
         "BV": synth.normal((H,), 44, 0.0, 0.1), "POS": synth.xavier(S, H, 45),
         "W1": synth.xavier(H, F, 46), "B1": synth.normal((F,), 47, 0.0, 0.1),
         "W2": synth.xavier(F, H, 48), "B2": None, "WO": synth.xavier(H, O, 49),
         "BO": synth.normal((O,), 50, 0.0, 0.1)}
    cur, blocks = ock.Cursor(), []
    models["transformer_rms"] = ("transformer", (dict(p), 0, 1),
                                 ock.transformer_meta(p, 0, 1, cur, blocks), blocks, cur.position)
    q = dict(p, G1=synth.normal((H,), 51, 1.0, 0.1), BE1=synth.normal((H,), 52, 0.0, 0.1),
             G2=synth.normal((H,), 53, 1.0, 0.1), BE2=synth.normal((H,), 54, 0.0, 0.1))
    cur, blocks = ock.Cursor(), []
    models["transformer_layer"] = ("transformer", (q, 1, 3),
                                   ock.transformer_meta(q, 1, 3, cur, blocks), blocks,
                                   cur.position)
    return models


@pytest.mark.gpu
def test_cpp_get_meta_data_and_get_data_match_oracle(tmp_path):
    """get_meta_data / get_data of Linear, MlpExecutor, InferenceMLP,
    TrainingMlp and the three transformer types (linear.rs:97-114,
    mlp.rs:99-119, 186-192, 221-228, encoder.rs:45-52, 90-110,
    decoder.rs:42-49).  Each model is loaded in the C++ program from a
    checkpoint the oracle wrote; its metadata must equal the oracle's
    cursor-built metadata field for field (byte ranges included), its
    cursor must end at the oracle's data_bytes, and get_data's blocks must
    be the oracle's parameters bit for bit."""
    import json

    from oracle import checkpoint as ock

    models = _oracle_models()
    for name, (kind, args, _, _, _) in models.items():
        path = str(tmp_path / name)
        if kind == "linear":
            ock.write_linear(path, *args)
        elif kind == "mlp":
            ock.write_mlp(path, *args)
        else:
            ock.write_transformer(path, *args)
    print("[case] C++ API program --metadata", flush=True)
    res = subprocess.run([BIN, "--metadata", str(tmp_path)], capture_output=True, text=True,
                         timeout=100)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    variants = {"linear": ["Linear"], "mlp": ["MlpExecutor", "InferenceMLP", "TrainingMlp"],
                "transformer": ["encoder.InferenceTransformer", "encoder.TrainingTransformer",
                                "decoder.InferenceTransformer"]}
    checked = 0
    for name, (kind, _, meta, blocks, data_bytes) in models.items():
        want = np.concatenate([np.asarray(b, np.float32).ravel() for b in blocks])
        for v in variants[kind]:
            with open(tmp_path / f"{name}.{v}.json") as f:
                got = json.load(f)
            assert got["meta"] == meta, (name, v)
            assert got["data_bytes"] == data_bytes == want.nbytes, (name, v)
            data = np.fromfile(tmp_path / f"{name}.{v}.f32", np.float32)
            assert data.shape == want.shape and np.array_equal(data.view(np.uint32),
                                                               want.view(np.uint32)), (name, v)
            checked += 1
    assert checked == 2 + 3 + 6
