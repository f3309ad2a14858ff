"""The Rust binding a maintainer would add to the reference (the one
`extern "C"` block of src/cuda/ffi.rs in the repository's integration notes)
checked against the C headers it binds, include/oxforge.h and
include/oxforge_net.h.

No Rust toolchain exists in this image, so the block is never compiled here;
this test is what keeps it true.  Both sides are parsed into canonical type
tokens and compared:
  - every function the headers declare has a `pub fn` of the same name, and
    the block declares nothing else;
  - arities match, and each parameter's type maps exactly (pointer depth and
    const-ness, the struct passed by value, the integer width, f32, c_int for
    the C enums), as does the return type;
  - the #[repr(C)] structs list the C structs' fields in the same order with
    the same types.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "oxforge.h"),
           os.path.join(ROOT, "include", "oxforge_net.h")]
DOC = os.path.join(ROOT, "INTEGRATION.md")

# C struct / handle name -> Rust name.
C_TYPES = {
    "forge_runtime": "ForgeRuntime", "forge_stream": "ForgeStream", "forge_event": "ForgeEvent",
    "forge_net_model": "ForgeModel", "forge_slice": "ForgeSlice",
    "forge_slice_u32": "ForgeSliceU32", "forge_gemm_epilogue": "ForgeGemmEpilogue",
    "forge_gemm_problem": "ForgeGemmProblem", "forge_transformer_desc": "ForgeTransformerDesc",
}
# C scalar -> canonical token (the C enums are passed as int).
C_SCALARS = {
    "size_t": "usize", "int": "c_int", "float": "f32", "uint32_t": "u32", "uint64_t": "u64",
    "long": "c_long", "char": "c_char", "void": "c_void", "forge_status": "Status",
    "forge_binary_op": "c_int", "forge_map_op": "c_int", "forge_activation": "c_int",
}
STRUCTS = ["forge_slice", "forge_slice_u32", "forge_gemm_epilogue", "forge_gemm_problem",
           "forge_transformer_desc"]


def _strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def c_type(decl):
    """Canonical token of a C parameter or return declaration, name removed:
    pointers become '*mut ' / '*const ' prefixes read from the outside in."""
    decl = " ".join(decl.replace("*", " * ").split())
    words = decl.split(" ")
    # Drop the parameter name (last identifier after the type and stars).
    if len(words) > 1 and words[-1] not in ("*", "const") and (
            words[-2] == "*" or words[-2] in C_SCALARS or words[-2] in C_TYPES):
        words = words[:-1]
    base_const = False
    base = None
    i = 0
    while i < len(words) and words[i] != "*":
        if words[i] == "const":
            base_const = True
        elif words[i] != "struct":
            base = words[i]
        i += 1
    tok = C_TYPES.get(base) or C_SCALARS.get(base)
    assert tok, f"unknown C type {base!r} in {decl!r}"
    # Each '*' wraps; a 'const' right after a '*' makes that pointer const.
    ptrs = []
    rest = words[i:]
    j = 0
    while j < len(rest):
        assert rest[j] == "*", decl
        const_ptr = j + 1 < len(rest) and rest[j + 1] == "const"
        ptrs.append(const_ptr)
        j += 2 if const_ptr else 1
    # The pointee's const-ness decides the innermost pointer's mutability;
    # for outer pointers, the constness of the pointer they point to.
    out = tok
    inner_const = base_const
    for const_ptr in ptrs:
        out = ("*const " if inner_const else "*mut ") + out
        inner_const = const_ptr
    return out


def c_functions():
    funcs = {}
    for path in HEADERS:
        text = _strip_comments(open(path).read())
        for m in re.finditer(r"(forge_status|const\s+char\s*\*)\s*(forge_\w+)\s*\(([^;]*?)\)\s*;",
                             text, re.S):
            ret, name, args = m.group(1), m.group(2), m.group(3)
            params = [a.strip() for a in args.split(",")] if args.strip() not in ("", "void") \
                else []
            funcs[name] = (c_type(ret), [c_type(p) for p in params])
    return funcs


def c_structs():
    structs = {}
    text = _strip_comments(open(HEADERS[0]).read() + open(HEADERS[1]).read())
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", text, re.S):
        fields = []
        for decl in m.group(2).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            # "size_t seq, hidden, ffn, out" declares several fields.
            head, *more = [d.strip() for d in decl.split(",")]
            first = head.split(" ")[-1].lstrip("*")
            base = head[: len(head) - len(first)].strip()
            for name in [first] + more:
                fields.append((name.lower(), c_type(base + " " + name)))
        structs[m.group(3)] = fields
    return structs


def rust_block():
    text = open(DOC).read()
    blocks = re.findall(r"```rust\n(.*?)```", text, re.S)
    ffi = [b for b in blocks if 'extern "C"' in b]
    assert len(ffi) == 1, "INTEGRATION.md should hold one extern \"C\" block"
    return re.sub(r"//[^\n]*", " ", ffi[0])


def rust_type(t):
    t = " ".join(t.split())
    out = ""
    while True:
        m = re.match(r"\*(mut|const)\s+(.*)", t)
        if not m:
            break
        out += f"*{m.group(1)} "
        t = m.group(2)
    return out + t


def rust_functions():
    body = rust_block()
    start = body.index('extern "C"')
    ext = body[start:body.index("\n}\n", start)]
    funcs = {}
    for m in re.finditer(r"pub\s+fn\s+(\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", ext, re.S):
        name, args, ret = m.group(1), m.group(2), m.group(3)
        params = []
        for a in [x.strip() for x in args.split(",") if x.strip()]:
            _, t = a.split(":", 1)
            params.append(rust_type(t))
        funcs[name] = (rust_type(ret) if ret else "()", params)
    return funcs


def rust_structs():
    body = rust_block()
    structs = {}
    for m in re.finditer(r"pub\s+struct\s+(\w+)\s*\{(.*?)\}", body, re.S):
        fields = []
        for f in [x.strip() for x in m.group(2).split(",") if x.strip()]:
            f = re.sub(r"^pub\s+", "", f)
            name, t = f.split(":", 1)
            fields.append((name.strip().lower(), rust_type(t)))
        structs[m.group(1)] = fields
    return structs


def test_c_parser_reads_known_prototypes():
    """The parser itself, on prototypes whose mapping is known by hand."""
    assert c_type("forge_runtime *rt") == "*mut ForgeRuntime"
    assert c_type("forge_stream *const *streams") == "*const *mut ForgeStream"
    assert c_type("forge_stream **out") == "*mut *mut ForgeStream"
    assert c_type("const forge_slice *params") == "*const ForgeSlice"
    assert c_type("const char *path") == "*const c_char"
    assert c_type("forge_slice x") == "ForgeSlice"
    assert c_type("size_t n") == "usize"
    assert c_type("forge_map_op op") == "c_int"
    assert c_type("uint64_t *data_bytes") == "*mut u64"
    f = c_functions()
    assert f["forge_gemm_f32"] == ("Status", ["*mut ForgeRuntime", "*mut ForgeStream", "ForgeSlice",
                                             "ForgeSlice", "ForgeSlice", "usize", "usize", "usize"])
    assert f["forge_last_error"] == ("*const c_char", [])


def test_every_header_function_is_bound_with_matching_types():
    c = c_functions()
    r = rust_functions()
    assert len(c) >= 85
    missing = sorted(set(c) - set(r))
    extra = sorted(set(r) - set(c))
    assert not missing, f"declared in include/*.h but not in the Rust block: {missing}"
    assert not extra, f"in the Rust block but not in include/*.h: {extra}"
    bad = {}
    for name, (ret, params) in c.items():
        rret, rparams = r[name]
        if len(params) != len(rparams):
            bad[name] = f"arity {len(params)} vs {len(rparams)}"
        elif params != rparams or ret != rret:
            bad[name] = [(a, b) for a, b in zip([ret] + params, [rret] + rparams) if a != b]
    assert not bad, bad


@pytest.mark.parametrize("c_name", STRUCTS)
def test_repr_c_structs_match_field_order(c_name):
    c = c_structs()[c_name]
    r = rust_structs()[C_TYPES[c_name]]
    assert c == r, (c_name, c, r)
