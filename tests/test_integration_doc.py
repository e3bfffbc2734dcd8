"""The Rust side of the drop-in (rust/: the mitten-kv-sys and mitten-kvhost-sys
FFI crates and the mitten-kv crate with the engine's PagedBackend, which a
maintainer adds to the engine's workspace next to
inference-backend/src/backend.rs:16-26) stays in step with the C ABI.

There is no Rust toolchain here to compile the crates, so the checks parse the
sources: every function of include/mitten_kv.h and include/mitten_kv_host.h is
declared in the FFI crates with the same parameter types and nothing else;
their constants equal the headers'; every FFI call in mitten-kv names a
declared function with its number of arguments; the backend implements the
engine's traits with the reference's method signatures; the manifests link
the libraries the build produces. CPU only."""
from __future__ import annotations

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUST = os.path.join(ROOT, "rust")
CRATES = {"mitten-kv-sys": ("mitten_kv.h", "MKV_API", "sys"),
          "mitten-kvhost-sys": ("mitten_kv_host.h", "MKVH_API", "hsys")}

_BASE = {"int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64", "uint16_t": "u16",
         "int": "i32", "float": "f32", "double": "f64", "void": "c_void", "char": "c_char"}


def _read(*parts) -> str:
    with open(os.path.join(*parts)) as f:
        return f.read()


def c_prototypes(path: str, macro: str):
    """[(name, return type, [(param type, param name)])] of the header's
    `macro`-marked declarations, in order."""
    text = re.sub(r"/\*.*?\*/", " ", _read(path), flags=re.S)
    out = []
    for m in re.finditer(macro + r"\s+([\w\s\*]+?)\s*\b(\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        ret, name, args = " ".join(m.group(1).split()), m.group(2), " ".join(m.group(3).split())
        params = []
        if args and args != "void":
            for a in args.split(","):
                pm = re.match(r"(.*?)(\w+)$", a.strip())
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
    b = _BASE.get(base[-1], base[-1])
    if stars == 0:
        return "()" if b == "c_void" else b
    if stars == 1 and b == "c_void" and pname == "stream" and not const:
        return "hipStream_t"
    if stars == 1:
        return f"*{'const' if const else 'mut'} {b}"
    if stars == 2:
        return f"*mut *{'const' if const else 'mut'} {b}"
    raise ValueError(ctype)


def rust_decls(src: str):
    """{name: ([param types], return type)} of the `extern "C"` block."""
    j = src.index('extern "C" {')
    body = re.sub(r"//[^\n]*", "", src[j:src.index("\n}\n", j)])
    out = {}
    for m in re.finditer(r"pub fn (\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", body, flags=re.S):
        args = [a.strip() for a in m.group(2).split(",") if a.strip()]
        out[m.group(1)] = ([" ".join(a.split(":", 1)[1].split()) for a in args],
                           " ".join((m.group(3) or "()").split()))
    return out


def _c_value(expr: str) -> int:
    """An integer constant: a literal (decimal or hex, C suffixes u / ull
    allowed, Rust digit separators) or `a << b` of two, in parentheses or not."""
    e = re.sub(r"(?<=[0-9A-Fa-f])(ull|ul|u)\b", "", expr.strip()).strip("() ").replace("_", "")
    parts = [int(x.strip("() "), 0) for x in e.split("<<")]
    if len(parts) == 1:
        return parts[0]
    if len(parts) == 2:
        return parts[0] << parts[1]
    raise ValueError(expr)


def c_constants(path: str) -> dict:
    """MKV_* / MKVH_* enumerators and #defines of a header, as integers."""
    text = re.sub(r"/\*.*?\*/", " ", _read(path), flags=re.S)
    out = {}
    for m in re.finditer(r"#define\s+(MKVH?_[A-Z0-9_]+)\s+(\(?[0-9][^\n]*)", text):
        out[m.group(1)] = _c_value(m.group(2))
    for body in re.findall(r"\benum\s*\{(.*?)\}", text, flags=re.S):
        for m in re.finditer(r"(MKVH?_[A-Z0-9_]+)\s*=\s*([^,}]+)", body):
            out[m.group(1)] = _c_value(m.group(2))
    return out


def rust_constants(src: str) -> dict:
    return {m.group(1): _c_value(m.group(2)) for m in re.finditer(r"pub const (\w+):\s*\w+\s*=\s*([^;]+);", src)}


def ffi_calls(src: str, alias: str):
    """[(name, argument count)] of every `alias::name(...)` call: the text
    between the balanced parentheses, split at its top-level commas."""
    out = []
    for m in re.finditer(rf"\b{alias}::(mkvh?_\w+)\s*\(", src):
        depth, i, pieces, cur = 1, m.end(), [], ""
        while True:
            c = src[i]
            i += 1
            depth += (c in "([{") - (c in ")]}")
            if depth == 0:
                break
            if depth == 1 and c == ",":
                pieces.append(cur)
                cur = ""
            else:
                cur += c
        pieces.append(cur)
        out.append((m.group(1), sum(1 for p in pieces if p.strip())))
    return out


@pytest.mark.parametrize("crate", list(CRATES))
def test_rust_extern_block_mirrors_the_header(crate):
    header, macro, _ = CRATES[crate]
    protos = c_prototypes(os.path.join(ROOT, "include", header), macro)
    assert len(protos) > 20
    decls = rust_decls(_read(RUST, crate, "src", "lib.rs"))
    names = [p[0] for p in protos]
    assert sorted(decls) == sorted(names), (
        f"missing in {crate}: {sorted(set(names) - set(decls))}; not in {header}: {sorted(set(decls) - set(names))}")
    for name, ret, params in protos:
        got, got_ret = decls[name]
        assert got == [rust_type(t, n) for t, n in params], f"{name}: {crate} has ({', '.join(got)})"
        assert got_ret == rust_type(ret, ""), f"{name}: return type {got_ret}"


@pytest.mark.parametrize("crate", list(CRATES))
def test_rust_constants_equal_the_header(crate):
    header = CRATES[crate][0]
    want = c_constants(os.path.join(ROOT, "include", header))
    got = rust_constants(_read(RUST, crate, "src", "lib.rs"))
    assert len(got) >= (20 if crate == "mitten-kv-sys" else 6)
    for name, value in got.items():
        assert name in want, f"{crate} defines {name}, which {header} does not"
        assert value == want[name], f"{name}: {crate} has {value}, {header} {want[name]}"
    status = [n for n in want if re.match(r"MKVH?_(OK|ERR_)", n)]
    assert set(status) <= set(got), f"{crate} lacks {sorted(set(status) - set(got))}"


def test_safe_crate_calls_declared_functions_with_their_arity():
    decls = {alias: rust_decls(_read(RUST, crate, "src", "lib.rs")) for crate, (_, _, alias) in CRATES.items()}
    srcdir = os.path.join(RUST, "mitten-kv", "src")
    seen = set()
    for fn in sorted(os.listdir(srcdir)):
        src = re.sub(r"//[^\n]*", "", _read(srcdir, fn))
        for alias, table in decls.items():
            for name, n in ffi_calls(src, alias):
                assert name in table, f"{fn}: {alias}::{name} is not declared"
                assert n == len(table[name][0]), f"{fn}: {alias}::{name} called with {n} arguments"
                seen.add(name)
    # The engine-facing path: the step, appends, extend, copies, plan and the lifecycle.
    for name in ("mkv_pool_create", "mkv_decode_plan_build_tables", "mkv_decode_step", "mkv_append_host",
                 "mkv_extend_attention_host", "mkv_copy_blocks_host", "mkv_pool_check", "mkvh_bm_admit",
                 "mkvh_bm_append", "mkvh_bm_schedule_prefill", "mkvh_bm_promote", "mkvh_bm_release",
                 "mkvh_bm_evict", "mkvh_bm_plan_compaction"):
        assert name in seen, f"mitten-kv never calls {name}"


# The engine's traits (inference-backend/src/backend.rs:16-26), method by method.
BACKEND_HANDLE = {
    "forward": "fn forward(&self, batch: &Batch) -> BoxFuture<'_, Result<Logits, EngineError>>",
    "kv_pool": "fn kv_pool(&self) -> &dyn KvPool",
    "model_config": "fn model_config(&self) -> &ModelConfig",
}
KV_POOL = {"free_pages": "fn free_pages(&self) -> usize", "total_pages": "fn total_pages(&self) -> usize"}


def _impl_body(src: str, header_re: str) -> str:
    m = re.search(header_re + r"[^{]*\{", src)
    assert m, header_re
    depth, i = 1, m.end()
    while depth:
        depth += {"{": 1, "}": -1}.get(src[i], 0)
        i += 1
    return src[m.end():i - 1]


@pytest.mark.parametrize("path,header,methods", [
    ("backend.rs", r"impl<M: PagedModel \+ 'static> BackendHandle for PagedBackend<M>", BACKEND_HANDLE),
    ("host.rs", r"impl KvPool for PoolView", KV_POOL),
])
def test_backend_implements_the_engine_traits(path, header, methods):
    body = " ".join(_impl_body(_read(RUST, "mitten-kv", "src", path), header).split())
    for name, sig in methods.items():
        assert sig in body, f"{path}: {name} is not `{sig}`"


def test_manifests_link_the_built_libraries():
    from mitten_amd import _build

    for crate, lib in (("mitten-kv-sys", _build.DEVICE_LIB), ("mitten-kvhost-sys", _build.HOST_LIB)):
        stem = os.path.basename(lib)[3:-3]  # libNAME.so
        assert f'name = "{crate}"' in _read(RUST, crate, "Cargo.toml")
        assert f"rustc-link-lib=dylib={stem}" in _read(RUST, crate, "build.rs")
    man = _read(RUST, "mitten-kv", "Cargo.toml")
    for dep in ("mitten-kv-sys", "mitten-kvhost-sys", "inference-backend"):
        assert re.search(rf"^{dep}\s*=", man, flags=re.M), f"mitten-kv does not depend on {dep}"
    lib = _read(RUST, "mitten-kv", "src", "lib.rs")
    for mod in ("backend", "error", "host", "pool"):
        assert f"mod {mod};" in lib and os.path.exists(os.path.join(RUST, "mitten-kv", "src", mod + ".rs"))


def test_the_checkers_see_drift():
    """A declaration with a wrong width, a call with one argument too few and
    a constant with another value all fail."""
    protos = {p[0]: p for p in c_prototypes(os.path.join(ROOT, "include", "mitten_kv.h"), "MKV_API")}
    _, _, params = protos["mkv_append"]
    drifted = ('extern "C" {\n    pub fn mkv_append(pool: *mut mkv_pool, layer: i32, k: *const c_void, '
               "v: *const c_void,\n        slots: *const i32, n: i64, stream: hipStream_t) -> i32;\n}\n")
    assert rust_decls(drifted)["mkv_append"][0] != [rust_type(t, n) for t, n in params]
    assert ffi_calls("sys::mkv_pool_check(self.raw, stream)", "sys") == [("mkv_pool_check", 2)]
    assert ffi_calls("sys::mkv_stream_synchronize(f(a, b))", "sys") == [("mkv_stream_synchronize", 1)]
    assert ffi_calls("sys::mkv_version()", "sys") == [("mkv_version", 0)]
    assert rust_constants("pub const MKV_ERR_HIP: i32 = 4;")["MKV_ERR_HIP"] != \
        c_constants(os.path.join(ROOT, "include", "mitten_kv.h"))["MKV_ERR_HIP"]
