"""The C++ drop-in API (include/oxforge_net.hpp: CudaRuntime, Matrix, Vector,
streams, the buffer pool, conversions, Linear, MLP) exercised on the GPU by
the in-tree program oxide-forge_amd/lib/oxforge_cpp_api_test, built from
oxide-forge_amd/csrc/tests/cpp_api_test.cpp by the same Makefile as the
library.  Its checks compare against host arithmetic: bit-exact for copies,
fills, conversions and single rounded elementwise ops, 1e-4 relative for the
GEMM, 1e-5 absolute for softmax and the norms."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oxide-forge_amd", "lib", "oxforge_cpp_api_test")


def test_cpp_api_program_is_built():
    assert os.path.exists(BIN), "run __graft_entry__.build() (make -C oxide-forge_amd/csrc)"


@pytest.mark.gpu
def test_cpp_api_on_gpu():
    print("[case] C++ API program", flush=True)
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=100)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "FAIL" not in res.stdout
