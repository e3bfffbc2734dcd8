"""The Rust FFI mirror in INTEGRATION.md (the mitten-kv-sys and
mitten-kvhost-sys extern blocks a maintainer would add to the engine's
workspace, next to inference-backend/src/backend.rs:16-26) declares every
function of include/mitten_kv.h and include/mitten_kv_host.h with the same
parameter types, and nothing else. CPU only: it parses the headers and the
document (there is no Rust toolchain here to compile the block)."""
from __future__ import annotations

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_BASE = {"int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64", "uint16_t": "u16",
         "int": "i32", "float": "f32", "double": "f64", "void": "c_void", "char": "c_char"}


def c_prototypes(path: str, macro: str):
    """[(name, return type, [(param type, param name)])] of the header's
    `macro`-marked declarations, in order."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    out = []
    for m in re.finditer(macro + r"\s+([\w\s\*]+?)\s*\b(\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        ret, name, args = " ".join(m.group(1).split()), m.group(2), " ".join(m.group(3).split())
        params = []
        if args and args != "void":
            for a in args.split(","):
                a = a.strip()
                pm = re.match(r"(.*?)(\w+)$", a)
                params.append((" ".join(pm.group(1).replace("*", " * ").split()), pm.group(2)))
        out.append((name, ret, params))
    return out


def rust_type(ctype: str, pname: str) -> str:
    """The Rust FFI type of a C parameter (or return) type."""
    toks = ctype.replace("*", " * ").split()
    stars = toks.count("*")
    const = "const" in toks
    base = [t for t in toks if t not in ("const", "*", "struct")]
    if not base:
        raise ValueError(ctype)
    b = base[-1]
    b = _BASE.get(b, b)
    if stars == 0:
        return "()" if b == "c_void" else b
    if stars == 1 and b == "c_void" and pname == "stream" and not const:
        return "hipStream_t"
    if stars == 1:
        return f"*{'const' if const else 'mut'} {b}"
    if stars == 2:
        return f"*mut *{'const' if const else 'mut'} {b}"
    raise ValueError(ctype)


def rust_decls(md_text: str, crate: str):
    """{name: [param types], return} from the `extern "C"` block that follows
    the crate's heading."""
    i = md_text.index(crate)
    j = md_text.index('extern "C" {', i)
    k = md_text.index("\n}\n", j)
    body = md_text[j:k]
    body = re.sub(r"//[^\n]*", "", body)
    out = {}
    for m in re.finditer(r"pub fn (\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", body, flags=re.S):
        args = [a.strip() for a in m.group(2).split(",") if a.strip()]
        types = [" ".join(a.split(":", 1)[1].split()) for a in args]
        out[m.group(1)] = (types, " ".join((m.group(3) or "()").split()))
    return out


@pytest.mark.parametrize("header,macro,crate", [("mitten_kv.h", "MKV_API", "mitten-kv-sys/src/lib.rs"),
                                                ("mitten_kv_host.h", "MKVH_API", "mitten-kvhost-sys/src/lib.rs")])
def test_rust_extern_block_mirrors_the_header(header, macro, crate):
    protos = c_prototypes(os.path.join(ROOT, "include", header), macro)
    assert len(protos) > 20
    md = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    decls = rust_decls(md, crate)
    names = [p[0] for p in protos]
    assert sorted(decls) == sorted(names), (
        f"missing in INTEGRATION.md: {sorted(set(names) - set(decls))}; "
        f"not in {header}: {sorted(set(decls) - set(names))}")
    for name, ret, params in protos:
        want = [rust_type(t, n) for t, n in params]
        got, got_ret = decls[name]
        assert got == want, f"{name}: INTEGRATION.md has ({', '.join(got)}), the header gives ({', '.join(want)})"
        assert got_ret == rust_type(ret, ""), f"{name}: return type {got_ret}"


def test_the_checker_sees_a_drifted_declaration():
    """A declaration with one parameter too few, or a wrong width, fails."""
    md = ('mitten-kv-sys/src/lib.rs\nextern "C" {\n'
          "    pub fn mkv_append(pool: *mut mkv_pool, layer: i32, k: *const c_void, v: *const c_void,\n"
          "                      slots: *const i32, n: i64, stream: hipStream_t) -> i32;\n}\n")
    protos = {p[0]: p for p in c_prototypes(os.path.join(ROOT, "include", "mitten_kv.h"), "MKV_API")}
    _, ret, params = protos["mkv_append"]
    got, _ = rust_decls(md, "mitten-kv-sys/src/lib.rs")["mkv_append"]
    assert got != [rust_type(t, n) for t, n in params]
