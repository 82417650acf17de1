"""The Rust -sys declarations (bindings/rust/src/lib.rs) against the C headers (include/mrun_moe.h,
include/mrun_load.h): the same functions, each with the same argument and return types in order,
the same struct fields in order, the same status codes. There is no Rust toolchain in this image,
so the declarations are parsed, not compiled."""
from __future__ import annotations

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
HEADERS = [ROOT / "include" / "mrun_moe.h", ROOT / "include" / "mrun_load.h"]
RUST = ROOT / "bindings" / "rust" / "src" / "lib.rs"

# C scalar type -> the Rust type the binding must use
C_SCALARS = {
    "int": "c_int", "int32_t": "i32", "int64_t": "i64", "uint32_t": "u32", "uint64_t": "u64",
    "size_t": "usize",
    "float": "f32", "char": "c_char", "void": "c_void", "uint16_t": "u16",
    "mrun_bf16": "mrun_bf16", "mrun_stream_t": "mrun_stream_t", "mrun_quantized": "mrun_quantized",
    "mrun_linear": "mrun_linear", "mrun_moe_config": "mrun_moe_config",
    "mrun_sparse_moe": "mrun_sparse_moe", "mrun_weights": "mrun_weights",
}


def c_type_to_rust(decl: str) -> str:
    """A C type (without the name) as the Rust type: `const T *` -> `*const T`, `T **` -> `*mut *mut
    T`, `const T *const *` -> `*const *const T`."""
    s = decl.replace("*", " * ").split()
    base_const = False
    toks = []
    for t in s:
        if t == "const" and not toks:
            base_const = True
        elif t == "const":
            toks.append("const")
        else:
            toks.append(t)
    base = C_SCALARS[toks[0]]
    # pointers, innermost first: qualifiers after each '*' apply to that pointer
    ptrs = []  # list of bool: is this pointer level itself const
    i = 1
    while i < len(toks):
        assert toks[i] == "*", decl
        c = i + 1 < len(toks) and toks[i + 1] == "const"
        ptrs.append(c)
        i += 2 if c else 1
    if not ptrs:
        return "()" if base == "c_void" else base
    out = f"*{'const' if base_const else 'mut'} {base}"
    for lvl in range(1, len(ptrs)):
        out = f"*{'const' if ptrs[lvl - 1] else 'mut'} {out}"
    return out


def c_functions() -> dict[str, tuple[str, list[str]]]:
    fns = {}
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"#.*", "", text)
        for m in re.finditer(r"([\w\s\*]+?)\b(mrun_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
            ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
            ret = ret.split("\n")[-1].strip()
            arg_types = []
            if args != "void":
                for a in args.split(","):
                    a = " ".join(a.split())
                    am = re.match(r"(.*?)(\w+)$", a)
                    arg_types.append(c_type_to_rust(am.group(1)))
            fns[name] = (c_type_to_rust(ret), arg_types)
    return fns


def rust_functions() -> dict[str, tuple[str, list[str]]]:
    text = re.sub(r"//.*", "", RUST.read_text())
    fns = {}
    for m in re.finditer(r"pub fn (\w+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", text, flags=re.S):
        name, args, ret = m.group(1), m.group(2), (m.group(4) or "()").strip()
        types = []
        for a in [x for x in args.split(",") if x.strip()]:
            types.append(" ".join(a.split(":", 1)[1].split()))
        fns[name] = (" ".join(ret.split()), types)
    return fns


def c_structs() -> dict[str, list[tuple[str, str]]]:
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "mrun_moe.h").read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef struct (\w+) \{(.*?)\} \1;", text, flags=re.S):
        fields = []
        for line in m.group(2).split(";"):
            line = " ".join(line.split())
            if not line:
                continue
            fm = re.match(r"(.*?)(\w+(?:\s*,\s*\w+)*)$", line)
            ty, names = fm.group(1).strip(), [n.strip() for n in fm.group(2).split(",")]
            # "int32_t experts, out, in" : the type is the first token group
            if "," in line and not ty:
                raise AssertionError(line)
            for n in names:
                fields.append((n, c_type_to_rust(ty)))
        out[m.group(1)] = fields
    return out


def rust_structs() -> dict[str, list[tuple[str, str]]]:
    text = re.sub(r"//.*", "", RUST.read_text())
    out = {}
    for m in re.finditer(r"pub struct (\w+) \{(.*?)\}", text, flags=re.S):
        fields = []
        for f in m.group(2).split(","):
            f = " ".join(f.split())
            if f.startswith("pub "):
                n, t = f[4:].split(":", 1)
                fields.append((n.strip().rstrip("_") if n.strip() == "in_" else n.strip(), t.strip()))
        out[m.group(1)] = fields
    return out


def test_every_c_function_is_declared_alike():
    c, r = c_functions(), rust_functions()
    assert len(c) >= 30
    assert set(c) == set(r), (set(c) ^ set(r))
    for name in c:
        assert c[name] == r[name], f"{name}: C {c[name]} vs Rust {r[name]}"


def test_structs_have_the_same_fields_in_order():
    c, r = c_structs(), rust_structs()
    assert set(c) == {"mrun_quantized", "mrun_linear", "mrun_moe_config", "mrun_sparse_moe"}
    for name, fields in c.items():
        assert fields == r[name], f"{name}: C {fields} vs Rust {r[name]}"
    assert r["mrun_weights"] == [], "mrun_weights stays opaque"


def test_status_codes_agree():
    h = (ROOT / "include" / "mrun_moe.h").read_text()
    c = dict((n, int(v)) for n, v in re.findall(r"(MRUN_\w+) = (\d+)", h))
    r = dict((n, int(v)) for n, v in re.findall(r"pub const (MRUN_\w+): c_int = (\d+);", RUST.read_text()))
    assert c == r and len(c) == 5


def test_type_mapping_examples():
    assert c_type_to_rust("const mrun_bf16 *") == "*const mrun_bf16"
    assert c_type_to_rust("mrun_weights **") == "*mut *mut mrun_weights"
    assert c_type_to_rust("const mrun_bf16 *const *") == "*const *const mrun_bf16"
    assert c_type_to_rust("const mrun_bf16 **") == "*mut *const mrun_bf16"
    assert c_type_to_rust("void *") == "*mut c_void"
    assert c_type_to_rust("void") == "()"


def test_manifest_with_links_has_a_build_script():
    """Cargo rejects a manifest that declares `links` without a build script; the script must name
    the library the `links` key declares."""
    manifest = (ROOT / "bindings" / "rust" / "Cargo.toml").read_text()
    m = re.search(r'^links\s*=\s*"([^"]+)"', manifest, flags=re.M)
    if m is None:
        return
    script = ROOT / "bindings" / "rust" / re.search(r'^build\s*=\s*"([^"]+)"', manifest, flags=re.M).group(1) \
        if re.search(r'^build\s*=', manifest, flags=re.M) else ROOT / "bindings" / "rust" / "build.rs"
    assert script.exists(), "links without a build script"
    text = script.read_text()
    assert f"cargo:rustc-link-lib=dylib={m.group(1)}" in text
    assert "fn main()" in text
