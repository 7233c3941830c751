"""The reference-side bindings against the C header they bind.

INTEGRATION.md documents the Rust shim a maintainer adds in place of the reference's src/engine.rs
(its `#[repr(C)]` structs mirror `model::Config`, `Tensor` and `Embed`, src/model.rs:22-103, and its
`extern "C"` block the entry points of include/sdhip.h).  Rust is not in this image, so nothing
compiles that shim; these tests parse it and check, against the header:
- every `#[repr(C)]` struct has the header struct's fields, in order, with the same C types;
- every `extern "C"` function has the header prototype's parameter and return types;
- every struct literal in the shim sets every field of its struct;
and that the ctypes structs of the Python binding have the header's layout as gcc compiles it
(sizeof and offsetof of every field).
"""
import ctypes as C
import importlib
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sdhip.h")
DOC = os.path.join(ROOT, "INTEGRATION.md")

C_BASE = {"size_t": "usize", "uint64_t": "u64", "uint32_t": "u32", "int32_t": "i32", "int": "i32",
          "uint8_t": "u8", "uint16_t": "u16", "double": "f64", "float": "f32", "char": "char", "void": "void",
          "sd_engine": "opaque", "sd_snapshot": "opaque", "sd_head": "opaque",
          "sd_config": "sd_config", "sd_tensor": "sd_tensor", "sd_embed": "sd_embed"}
RUST_BASE = {"usize": "usize", "u64": "u64", "u32": "u32", "i32": "i32", "c_int": "i32", "u8": "u8",
             "u16": "u16", "f64": "f64", "f32": "f32", "c_char": "char", "c_void": "void*",
             "SdConfig": "sd_config", "SdTensor": "sd_tensor", "SdEmbed": "sd_embed"}


def _strip_c_comments(s):
    s = re.sub(r"/\*.*?\*/", " ", s, flags=re.S)
    return re.sub(r"//[^\n]*", " ", s)


def c_type(decl):
    """Canonical form of a C type: a base name, or ("ptr", pointee_is_const, pointee)."""
    toks = re.findall(r"\w+|\*", decl)
    i = 0
    const = False
    base = None
    while i < len(toks) and toks[i] != "*":
        if toks[i] == "const":
            const = True
        elif toks[i] not in ("struct", "unsigned", "signed"):
            base = toks[i]
        i += 1
    assert base in C_BASE, f"unknown C type in {decl!r}"
    cur = C_BASE[base]
    while i < len(toks):
        assert toks[i] == "*", decl
        i += 1
        nxt_const = i < len(toks) and toks[i] == "const"
        if nxt_const:
            i += 1
        cur = ("ptr", const, cur)
        const = nxt_const
    return cur


def rust_type(decl):
    decl = decl.strip()
    m = re.match(r"\*(const|mut)\s+(.*)$", decl)
    if m:
        return ("ptr", m.group(1) == "const", rust_type(m.group(2)))
    assert decl in RUST_BASE, f"unknown Rust type {decl!r}"
    return RUST_BASE[decl]


def same(c, r):
    """C and Rust canonical types agree; Rust's c_void stands for void or an opaque handle."""
    if r == "void*":
        return c in ("void", "opaque")
    if isinstance(c, tuple) and isinstance(r, tuple):
        return c[1] == r[1] and same(c[2], r[2])
    return c == r


def header():
    text = _strip_c_comments(open(HEADER).read())
    structs = {}
    for body, name in re.findall(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        fields = []
        for stmt in body.split(";"):
            stmt = stmt.strip()
            if not stmt:
                continue
            # "T a, b, *c": the type is what precedes the first declarator
            m = re.match(r"((?:const\s+)?\w+(?:\s*\*\s*(?:const\s*)?)*)\s*(.*)$", stmt, flags=re.S)
            base, decls = m.group(1), m.group(2)
            for d in decls.split(","):
                d = d.strip()
                stars = d.count("*")
                name_ = d.replace("*", "").strip()
                fields.append((name_, c_type(base + " *" * stars)))
        structs[name] = fields
    funcs = {}
    for ret, name, params in re.findall(r"([\w\s\*]+?)\b(sd_\w+)\s*\(([^()]*)\)\s*;", text, flags=re.S):
        ret = ret.strip().split("\n")[-1].strip()
        ps = []
        for p in params.split(","):
            p = p.strip()
            if not p or p == "void":
                continue
            m = re.match(r"(.*?)(\w+)\s*$", p, flags=re.S)
            ps.append(c_type(m.group(1)))
        funcs[name] = (c_type(ret) if ret != "void" else None, ps)
    return structs, funcs


def rust_blocks():
    return re.findall(r"```rust\n(.*?)```", open(DOC).read(), flags=re.S)


def shim():
    structs, funcs, literals = {}, {}, []
    for code in rust_blocks():
        for name, body in re.findall(r"#\[repr\(C\)\]\s*struct\s+(\w+)\s*\{(.*?)\}", code, flags=re.S):
            fields = []
            for f in body.split(","):
                f = f.strip()
                if f:
                    n, t = f.split(":", 1)
                    fields.append((n.strip(), rust_type(t)))
            structs[name] = fields
        for block in re.findall(r'extern\s+"C"\s*\{(.*?)\n\}', code, flags=re.S):
            for name, params, ret in re.findall(r"fn\s+(\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
                ps = []
                for p in params.split(","):
                    p = p.strip()
                    if p:
                        ps.append(rust_type(p.split(":", 1)[1]))
                funcs[name] = (rust_type(ret) if ret else None, ps)
        for m in re.finditer(r"\b(Sd[A-Z]\w*)\s*\{((?:[^{}]|\{[^{}]*\})*)\}", code):
            if re.search(r"struct\s+$", code[:m.start()]):
                continue  # the definition itself
            keys = re.findall(r"(?:^|,)\s*(\w+)\s*:", m.group(2))
            literals.append((m.group(1), keys))
    return structs, funcs, literals


RUST_TO_C = {"SdConfig": "sd_config", "SdTensor": "sd_tensor", "SdEmbed": "sd_embed"}


def test_shim_structs_match_header():
    hs, _ = header()
    rs, _, _ = shim()
    assert set(RUST_TO_C) <= set(rs), f"the shim defines {sorted(rs)}"
    for rname, cname in RUST_TO_C.items():
        cf, rf = hs[cname], rs[rname]
        assert len(rf) == len(cf), f"{rname}: {len(rf)} fields, {cname} has {len(cf)} ({[n for n, _ in cf]})"
        for (cn, ct), (rn, rt) in zip(cf, rf):
            assert same(ct, rt), f"{rname}.{rn} is {rt}, {cname}.{cn} is {ct}"


def test_shim_functions_match_header():
    _, hf = header()
    _, rf, _ = shim()
    assert len(rf) >= 9, f"only {sorted(rf)} declared"
    for name, (rret, rps) in rf.items():
        assert name in hf, f"{name} is not in include/sdhip.h"
        cret, cps = hf[name]
        assert len(rps) == len(cps), f"{name}: {len(rps)} parameters, the header has {len(cps)}"
        for i, (ct, rt) in enumerate(zip(cps, rps)):
            assert same(ct, rt), f"{name} parameter {i}: shim {rt}, header {ct}"
        assert (cret is None) == (rret is None) and (cret is None or same(cret, rret)), f"{name}: return type"


def test_shim_struct_literals_set_every_field():
    rs, _, lits = shim()
    seen = {n for n, _ in lits}
    assert {"SdConfig", "SdTensor", "SdEmbed"} <= seen, f"literals found: {sorted(seen)}"
    for name, keys in lits:
        want = [n for n, _ in rs[name]]
        assert sorted(keys) == sorted(want), f"{name} literal sets {keys}, the struct has {want}"


def test_parser_catches_a_short_struct():
    """The check is not vacuous: the struct the round-trip found short is reported."""
    hs, _ = header()
    short = [("rows_path", rust_type("*const c_char")), ("vocab", "u64"), ("row_bytes", "u64"),
             ("n_parts", "usize"), ("part_names", rust_type("*const *const c_char")),
             ("part_bytes", rust_type("*const u64"))]
    assert len(short) != len(hs["sd_embed"])
    swapped = [("a", "u32")] + [(n, t) for n, t in short]
    assert not all(same(c, r) for (_, c), (_, r) in zip(hs["sd_embed"], swapped))
    # const-ness of a pointee is part of the type
    assert not same(c_type("const char* const*"), rust_type("*const *mut c_char"))
    assert same(c_type("sd_engine**"), rust_type("*mut *mut c_void"))
    assert same(c_type("const char**"), rust_type("*mut *const c_char"))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is needed to measure the header's layout")
def test_python_structs_have_the_header_layout(tmp_path):
    hs, _ = header()
    src = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, fields in hs.items():
        src.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for n, _ in fields:
            src.append(f'printf("{cname}.{n} %zu\\n", offsetof({cname}, {n}));')
    src.append("return 0; }")
    (tmp_path / "layout.c").write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(tmp_path / "layout.c")], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                         text=True).stdout.splitlines())
    import sys
    sys.path.insert(0, ROOT)
    mod = importlib.import_module("strands-decider-rs_amd")
    for cname, fields in hs.items():
        py = getattr(mod, cname)
        assert C.sizeof(py) == int(got[cname]), cname
        assert [n for n, _ in py._fields_] == [n for n, _ in fields], cname
        for n, _ in fields:
            assert getattr(py, n).offset == int(got[f"{cname}.{n}"]), f"{cname}.{n}"
