"""The Rust FFI crate (rust/llmoxide-hip-ffi) against the C header it mirrors.

There is no Rust toolchain in this image, so the crate cannot be compiled here;
these tests keep it in step with include/lmx/attn.h instead: the same entry
points with the same parameter types in the same order, the same structs with
the same fields, and the same constants.  The struct sizes the crate's own
(cargo) test asserts are checked against the sizes a C compiler gives the
header's structs.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lmx", "attn.h")
CRATE = os.path.join(ROOT, "rust", "llmoxide-hip-ffi")
LIB_RS = os.path.join(CRATE, "src", "lib.rs")

BASE = {"void": "c_void", "char": "c_char", "float": "f32", "uint32_t": "u32", "int32_t": "i32",
        "int": "i32", "size_t": "usize", "lmx_status": "i32", "lmx_dtype": "i32",
        "lmx_stream": "HipStream"}


def rust_struct_name(c_name: str) -> str:
    return "".join(part.capitalize() for part in c_name.split("_"))  # lmx_kv_desc -> LmxKvDesc


def c_to_rust(ctype: str) -> str:
    """A C parameter or field type (no name) as the Rust type it must map to."""
    toks = re.findall(r"\w+|\*", ctype)
    base_const, i = False, 0
    while toks[i] == "const":
        base_const, i = True, i + 1
    base = toks[i]
    i += 1
    if i < len(toks) and toks[i] == "const":  # "float const *"
        base_const, i = True, i + 1
    ptr_consts = []
    while i < len(toks):
        assert toks[i] == "*", ctype
        i += 1
        c = i < len(toks) and toks[i] == "const"
        if c:
            i += 1
        ptr_consts.append(c)
    t = BASE.get(base) or rust_struct_name(base)
    pointee_const = base_const
    for c in ptr_consts:
        t = ("*const " if pointee_const else "*mut ") + t
        pointee_const = c
    return t


def strip_c_comments(s: str) -> str:
    return re.sub(r"/\*.*?\*/", "", s, flags=re.S)


def header_functions():
    h = strip_c_comments(open(HEADER).read())
    out = {}
    for ret, name, args in re.findall(r"^([a-z][\w \*]*?)\s*\b(lmx_\w+)\s*\(([^;]*?)\)\s*;", h, flags=re.M | re.S):
        params = []
        args = " ".join(args.split())
        if args != "void":
            for a in args.split(","):
                m = re.match(r"^(.*?)(\w+)$", a.strip())
                params.append((m.group(2), c_to_rust(m.group(1))))
        ret = " ".join(ret.split())
        out[name] = (params, None if ret == "void" else c_to_rust(ret))
    return out


def header_structs():
    h = strip_c_comments(open(HEADER).read())
    out = {}
    for body, name in re.findall(r"typedef struct \{(.*?)\}\s*(\w+);", h, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if decl:
                m = re.match(r"^(.*?)(\w+)$", decl)
                fields.append((m.group(2), c_to_rust(m.group(1))))
        out[rust_struct_name(name)] = fields
    return out


def header_constants():
    h = strip_c_comments(open(HEADER).read())
    out = {k: int(v) for k, v in re.findall(r"\b(LMX_\w+)\s*=\s*(\d+)", h)}
    for k, a, b in re.findall(r"#define\s+(LMX_\w+)\s+\((\d+)u\s*<<\s*(\d+)\)", h):
        out[k] = int(a) << int(b)
    return out


def rust_source():
    return re.sub(r"//[^\n]*", "", open(LIB_RS).read())


def rust_functions():
    src = rust_source()
    block = re.search(r'extern "C" \{(.*?)\n\}', src, flags=re.S).group(1)
    out = {}
    for name, args, ret in re.findall(r"pub fn (\w+)\((.*?)\)\s*(?:->\s*([^;]+?))?\s*;", block, flags=re.S):
        params = []
        args = " ".join(args.split())
        if args:
            for a in args.split(","):
                if a.strip():
                    pname, ptype = a.split(":", 1)
                    params.append((pname.strip(), " ".join(ptype.split())))
        out[name] = (params, " ".join(ret.split()) if ret else None)
    return out


def rust_structs():
    out = {}
    for name, body in re.findall(r"pub struct (\w+) \{(.*?)\}", rust_source(), flags=re.S):
        fields = re.findall(r"pub (?:r#)?(\w+): ([^,]+),", body)
        out[name] = [(n, " ".join(t.split())) for n, t in fields]
    return out


def rust_constants():
    out = {}
    for name, expr in re.findall(r"pub const (LMX_\w+): \w+ = ([^;]+);", rust_source()):
        m = re.match(r"^(\d+)\s*<<\s*(\d+)$", expr.strip())
        out[name] = int(m.group(1)) << int(m.group(2)) if m else int(expr)
    return out


def test_the_crate_declares_every_entry_point_of_the_header():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 30
    assert sorted(h) == sorted(r), (set(h) ^ set(r))


@pytest.mark.parametrize("name", sorted(header_functions()))
def test_entry_point_signature(name):
    h_params, h_ret = header_functions()[name]
    r_params, r_ret = rust_functions()[name]
    assert [t for _, t in r_params] == [t for _, t in h_params], (name, r_params, h_params)
    assert [n for n, _ in r_params] == [n for n, _ in h_params], name
    assert r_ret == h_ret, (name, r_ret, h_ret)


def test_structs_match_field_for_field():
    h, r = header_structs(), rust_structs()
    for name, fields in h.items():
        assert name in r, name
        assert r[name] == fields, (name, r[name], fields)


def test_constants_match():
    h, r = header_constants(), rust_constants()
    assert h, "no constants parsed from the header"
    for k, v in h.items():
        assert r.get(k) == v, (k, r.get(k), v)


def test_the_mapping_itself():
    # the few non-trivial cases of c_to_rust, checked by hand
    assert c_to_rust("const void *const *") == "*const *const c_void"
    assert c_to_rust("const void **") == "*mut *const c_void"
    assert c_to_rust("lmx_kvm **") == "*mut *mut LmxKvm"
    assert c_to_rust("const char *") == "*const c_char"
    assert c_to_rust("lmx_stream") == "HipStream"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs a C compiler")
def test_struct_sizes_the_crate_asserts_are_the_c_sizes(tmp_path):
    asserted = dict(re.findall(r"size_of::<(\w+)>\(\), (\d+)\)", open(LIB_RS).read()))
    c_names = {rust_struct_name(n): n for n in re.findall(r"\}\s*(lmx_\w+);",
                                                         strip_c_comments(open(HEADER).read()))}
    src = tmp_path / "sizes.c"
    src.write_text('#include <stdio.h>\n#include "lmx/attn.h"\nint main(void) {\n' +
                   "".join(f'  printf("{r} %zu\\n", sizeof({c_names[r]}));\n' for r in asserted) +
                   "  return 0;\n}\n")
    exe = tmp_path / "sizes"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                        check=True).stdout.splitlines())
    assert len(asserted) == len(header_structs())
    for name, size in asserted.items():
        assert got[name] == size, (name, got[name], size)
