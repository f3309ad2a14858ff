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
