"""CPU: the Rust FFI crate (qora-llm-4b_amd/rust/qora-mixer-sys) against the
C header it binds.  Rust is not installed here, so the crate is checked as
text: every function of include/qora_mixer.h is declared in the crate's
`extern "C"` block with the same name, the same number of arguments and
arguments of the same kind and width (pointer, i32, i64, u64, f32, f64), and
the same return type; every #[repr(C)] struct has the header struct's field
types in the same order; the status and flag constants agree; and build.rs
compiles the same kernel files with the same device flags as build.py.
"""
from __future__ import annotations

import re

from conftest import PKG, ROOT

HEADER = ROOT / "include" / "qora_mixer.h"
CRATE = PKG / "rust" / "qora-mixer-sys"

C_SCALARS = {"int32_t": "i32", "int64_t": "i64", "uint64_t": "u64", "float": "f32", "double": "f64",
             "void": "void", "qm_stream": "ptr"}
R_SCALARS = {"i32": "i32", "i64": "i64", "u64": "u64", "f32": "f32", "f64": "f64", "qm_stream": "ptr"}


def _strip_c_comments(text: str) -> str:
    return re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", text, flags=re.S))


def c_kind(decl: str) -> str:
    decl = decl.replace("const", " ").strip()
    if "*" in decl:
        return "ptr"
    base = decl.split()[0] if " " in decl else decl
    return C_SCALARS[base]


def r_kind(ty: str) -> str:
    ty = ty.strip()
    if ty.startswith("*"):
        return "ptr"
    return R_SCALARS[ty]


def header_functions() -> dict:
    text = _strip_c_comments(HEADER.read_text())
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(qm_\w+)\s*\(([^;{]*?)\)\s*;", text):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        ret = ret.split()[-1] if ret.split() else ret
        ret_kind = "ptr" if "*" in m.group(1) else C_SCALARS[ret.replace("*", "").strip()]
        params = [p.strip() for p in args.split(",") if p.strip() and p.strip() != "void"]
        kinds = []
        for p in params:
            # drop the parameter name: the last identifier
            ty = re.sub(r"\b\w+\s*$", "", p).strip()
            kinds.append(c_kind(ty))
        out[name] = (ret_kind, kinds)
    return out


def crate_functions() -> dict:
    text = (CRATE / "src" / "lib.rs").read_text()
    block = re.search(r'extern "C"\s*\{(.*?)\n    \}', text, flags=re.S).group(1)
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub fn (qm_\w+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        name, args, ret = m.group(1), m.group(2), m.group(4)
        kinds = [r_kind(a.split(":", 1)[1]) for a in args.split(",") if a.strip()]
        ret_kind = "void" if ret is None else r_kind(ret)
        out[name] = (ret_kind, kinds)
    return out


def test_crate_declares_every_header_function_with_matching_arguments():
    h, r = header_functions(), crate_functions()
    assert len(h) >= 40, sorted(h)
    assert set(h) == set(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name in h:
        assert h[name] == r[name], (name, h[name], r[name])


def _c_struct_fields(name: str) -> list[str]:
    text = _strip_c_comments(HEADER.read_text())
    m = re.search(r"typedef struct(?: \w+)?\s*\{([^{}]*)\}\s*" + name + r"\s*;", text)
    assert m, name
    return [c_kind(re.sub(r"\b\w+\s*$", "", f.strip())) for f in m.group(1).split(";") if f.strip()]


def _r_struct_fields(name: str) -> list[str]:
    text = (CRATE / "src" / "lib.rs").read_text()
    m = re.search(r"pub struct " + name + r"\s*\{(.*?)\n    \}", text, flags=re.S)
    assert m, name
    return [r_kind(f.split(":", 1)[1]) for f in m.group(1).split(",") if ":" in f]


def test_repr_c_structs_match_the_header():
    for s in ("qm_config", "qm_q4_out", "qm_sample_params"):
        assert _c_struct_fields(s) == _r_struct_fields(s), s


def test_constants_match_the_header():
    htext = HEADER.read_text()
    rtext = (CRATE / "src" / "lib.rs").read_text()
    consts = dict(re.findall(r"\b(QM_[A-Z0-9_]+)\s*=\s*(\d+)", htext))
    assert len(consts) >= 18
    for name, value in consts.items():
        m = re.search(r"pub const " + name + r":\s*i32\s*=\s*(\d+);", rtext)
        assert m and m.group(1) == value, name


def test_build_script_follows_the_python_recipe():
    import importlib.util
    spec = importlib.util.spec_from_file_location("qora_build_check", PKG / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    rs = (CRATE / "build.rs").read_text()
    kernels = re.search(r"const KERNELS: &\[&str\] = &\[(.*?)\];", rs, flags=re.S).group(1)
    assert re.findall(r'"(\w+)"', kernels) == list(b.KERNELS)
    flags = re.search(r"const HIPCC_FLAGS: &\[&str\] = &\[(.*?)\];", rs, flags=re.S).group(1)
    rflags = re.findall(r'"([^"]+)"', flags)
    assert rflags == [f for f in b.HIPCC_FLAGS if f != "--genco"]
    for needed in ("--genco", "qm_noalloc.hip", "qm_runtime.cpp", "-lamdhip64", "rustc-link-lib=dylib=qora_mixer"):
        assert needed in rs, needed
    cargo = (CRATE / "Cargo.toml").read_text()
    assert 'links = "qora_mixer"' in cargo and 'build = "build.rs"' in cargo


def test_layer_wrappers_are_unsafe_and_check_lengths():
    """The layer-forward wrappers hand raw device pointers to kernels, so
    they are `unsafe fn` with a `# Safety` section; lengths reach the C ABI
    through checked conversions (an oversized usize is an error, not a
    wrapped i32)."""
    text = (CRATE / "src" / "lib.rs").read_text()
    for fn in ("deltanet_decode", "attn_decode", "deltanet_prefill", "attn_prefill"):
        m = re.search(r"((?:///[^\n]*\n)+)pub (unsafe )?fn " + fn + r"\(", text)
        assert m and m.group(2), fn
        assert "# Safety" in m.group(1), fn
    body = text[text.index("pub use raw::"):]
    assert not re.search(r"\bas i32\b", body), "narrowing cast outside the raw declarations"
    assert "i32::try_from" in body and "i64::try_from" in body
