"""C ABI checks that need no GPU: the library loads, exports every entry
point include/oxforge.h declares, reports errors as status codes, and the
code object contains every kernel instance the host dispatcher can name."""
import ctypes
import os
import re

import pytest

import oxforge
from oxforge import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "oxforge.h")


def header_functions(path):
    text = open(path).read()
    return sorted(set(re.findall(r"^(?:forge_status|const char \*)\s*(forge_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = oxforge.load()
    names = header_functions(HEADER)
    assert len(names) >= 40
    for n in names:
        assert hasattr(lib, n), f"{n} declared in oxforge.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_executor_entry_points_exported():
    from oxforge import net

    lib = oxforge.load()
    names = header_functions(os.path.join(ROOT, "include", "oxforge_net.h"))
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), f"{n} declared in oxforge_net.h but not exported"
        assert n in net.SIGNATURES, f"{n} has no ctypes signature"


def test_status_strings_and_errors_without_device():
    lib = oxforge.load()
    assert lib.forge_status_string(0) == b"ok"
    assert lib.forge_status_string(1) == b"invalid argument"
    n = ctypes.c_int(-1)
    assert lib.forge_device_count(ctypes.byref(n)) == 0
    if n.value == 0:
        h = ctypes.c_void_p()
        st = lib.forge_runtime_create(0, None, ctypes.byref(h))
        assert st == _lib.FORGE_ENODEV
        assert b"device" in lib.forge_last_error()
        assert not h.value
    # null arguments are rejected with EINVAL, never a crash
    assert lib.forge_device_count(None) == _lib.FORGE_EINVAL
    assert lib.forge_sync(None, None) == _lib.FORGE_EINVAL
    assert lib.forge_alloc(None, 4, None) == _lib.FORGE_EINVAL
    assert lib.forge_gemm_f32(None, None, _lib.NULL_SLICE, _lib.NULL_SLICE, _lib.NULL_SLICE, 1, 1, 1) \
        == _lib.FORGE_EINVAL
    assert lib.forge_runtime_destroy(None) == 0


def dispatcher_kernel_names():
    """Every kernel name runtime.cpp can build (mirrors its naming rules)."""
    names = []
    tiles = ("128x128x32_x", "128x64x32_x", "64x128x32_x", "64x64x32_x")
    for ab in ("nn", "nt", "tn", "tt"):
        for tag in tiles + ("64x64x16_2x2_g",):
            names.append(f"forge_gemm_{ab}_{tag}_e")
        # row statistics / column sums instances of the unguarded tiles, and
        # the same with the row subtrahend
        for tag in tiles + ("64x128x32_x8",):
            names.append(f"forge_gemm_{ab}_{tag}_s")
            names.append(f"forge_gemm_{ab}_{tag}_r")
        # fused epilogue over K segments (forge_gemm_sum_f32)
        for tag in tiles:
            names.append(f"forge_gemm_{ab}_{tag}_k")
    for tag in tiles + ("128x256x32_x", "64x64x16_2x2_g"):
        names.append(f"forge_gemm_nn_{tag}")
    # batched (forge_gemm_batch_f32, Q/K/V and split-K slices): every layout
    for ab in ("nn", "nt", "tn", "tt"):
        for tag in tiles:
            names.append(f"forge_gemm_batch_{ab}_{tag}")
    # eight-wave 64x128 tile: plain NN, every epilogue kind, batched NN/NT/TN
    names.append("forge_gemm_nn_64x128x32_x8")
    names += [f"forge_gemm_{ab}_64x128x32_x8_e" for ab in ("nn", "nt", "tn", "tt")]
    names += [f"forge_gemm_batch_{ab}_64x128x32_x8" for ab in ("nn", "nt", "tn")]
    names += ["forge_gemm_splitk_reduce_v", "forge_gemm_splitk_reduce_s"]
    for op in ("softmax", "layer_norm", "rms_norm", "softmax_bwd", "layer_norm_bwd", "rms_norm_bwd"):
        for v in (1, 2, 4, 8, 16):
            names.append(f"forge_row_{op}_v{v}")
        names.append(f"forge_row_{op}_loop")
    for op in ("layer_norm_bwd", "rms_norm_bwd"):
        for v in (1, 2, 4, 8):
            names.append(f"forge_row_{op}_v{v}_p")
            names.append(f"forge_row_{op}_v{v}_p_d")
        for v in (1, 2, 4, 8, 16):
            names.append(f"forge_row_{op}_v{v}_d")
        names.append(f"forge_row_{op}_v4_p4")
        names.append(f"forge_row_{op}_v4_p4_d")
    for op in ("add", "sub", "mul", "div"):
        for k in ("binary", "binary_assign", "by_rows"):
            for s in ("v", "s"):
                names.append(f"forge_{k}_{op}_{s}")
    for op in ("scale", "add", "gelu", "gelu_d", "relu", "relu_d", "silu", "silu_d",
               "exp_shift", "half_sq", "identity"):
        names += [f"forge_map_{op}_v", f"forge_map_{op}_s", f"forge_map_sum_{op}",
                  f"forge_map_sum_{op}_v"]
    names += ["forge_fill_random", "forge_act_backward_v", "forge_act_backward_s",
              "forge_count_neq", "forge_count_final", "forge_count_neq_u32",
              "forge_count_final_u32", "forge_sgd_v", "forge_sgd_s", "forge_row_rms_parts",
              "forge_row_sq_parts"]
    names += ["forge_fill_v", "forge_fill_s", "forge_fill_seq", "forge_causal_mask",
              "forge_sum_cols_v", "forge_sum_cols_s", "forge_sum_cols_final", "forge_sum_cols_final2",
              "forge_sum_cols_final_v", "forge_sum_cols_final2_v",
              "forge_sum_cols_p4", "forge_sum_cols_p8", "forge_sum_cols_p16",
              "forge_sum_rows_v", "forge_sum_rows_s", "forge_reduce_sum", "forge_reduce_max",
              "forge_reduce_sum_v", "forge_reduce_max_v",
              "forge_transpose", "forge_transpose_w", "forge_transpose_g"]
    return names


def test_code_object_contains_dispatched_kernels():
    assert os.path.exists(_lib.KERNELS_PATH), "code object not built"
    blob = open(_lib.KERNELS_PATH, "rb").read()
    assert b"gfx950" in blob
    missing = [n for n in dispatcher_kernel_names() if (n.encode() + b"\0") not in blob]
    assert not missing, f"kernels missing from the code object: {missing}"


def test_runtime_source_names_only_known_kernels():
    src = open(os.path.join(ROOT, "oxide-forge_amd", "csrc", "runtime", "runtime.cpp")).read()
    literals = set(re.findall(r'"(forge_[a-z0-9_]+)"', src))
    known = set(dispatcher_kernel_names())
    assert literals <= known, f"unknown kernel literals: {literals - known}"


@pytest.mark.parametrize("fn", ["forge_alloc", "forge_softmax_rows", "forge_gemm_ex_f32"])
def test_signatures_declared(fn):
    assert fn in _lib.SIGNATURES


def test_code_object_kernels_do_not_spill():
    """No kernel of the built gfx950 code object spills registers or uses
    per-lane scratch: a spill in a row or GEMM kernel costs tens of percent
    (a norm backward at 8 float4 per lane that spilled 66 VGPRs ran at 38.7
    against 27.5 us).  Reads the code object's own metadata notes."""
    import subprocess
    import tempfile

    bundler = "/opt/rocm/llvm/bin/clang-offload-bundler"
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    if not (os.path.exists(bundler) and os.path.exists(readelf)):
        pytest.skip("ROCm LLVM tools not installed")
    assert os.path.exists(_lib.KERNELS_PATH), "code object not built"
    with tempfile.TemporaryDirectory() as d:
        obj = os.path.join(d, "k.o")
        subprocess.run([bundler, "--unbundle", "--type=o",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                        f"--input={_lib.KERNELS_PATH}", f"--output={obj}"], check=True)
        notes = subprocess.run([readelf, "--notes", obj], check=True, capture_output=True,
                               text=True).stdout
    bad, name, kernels = [], None, 0
    for line in notes.splitlines():
        key, _, value = line.strip().lstrip("- ").partition(":")
        value = value.strip()
        if key == ".name" and value.startswith("forge_"):
            name, kernels = value, kernels + 1
        elif name and key in (".vgpr_spill_count", ".sgpr_spill_count",
                              ".private_segment_fixed_size") and value.isdigit() and int(value):
            bad.append((name, key, int(value)))
    assert kernels > 100, kernels
    assert not bad, bad
