"""The Rust FFI crate (bindings/woolly-hip/src/lib.rs) against the C header.

There is no Rust toolchain here, so the crate is checked by parsing: every
WH_API function of include/woolly_hip.h is declared in the crate's extern "C"
block with the same name, arity and argument / return types (C types mapped to
their Rust FFI equivalents), every #[repr(C)] struct has the header's fields in
the header's order with matching types, every status / type / value-type
constant has the header's value, and the crate declares nothing the header
does not.  The reference binds the backend from Rust (north star: a thin
extern "C" FFI crate); tests/test_abi.py checks that the built library exports
the same symbols.
"""
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "woolly_hip.h"
CRATE = ROOT / "bindings" / "woolly-hip" / "src" / "lib.rs"

_C_BASE = {
    "int": "c_int", "size_t": "usize", "uint64_t": "u64", "uint32_t": "u32", "int32_t": "i32",
    "float": "c_float", "void": "c_void", "char": "c_char",
}


def _strip_c_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def _strip_rust_comments(text: str) -> str:
    return re.sub(r"//[^\n]*", " ", text)


def c_type_to_rust(ctype: str) -> str:
    """`const wh_weight**` -> `*mut *const wh_weight`, `size_t` -> `usize`, ..."""
    ctype = " ".join(ctype.split())
    stars = ctype.count("*")
    is_const = ctype.startswith("const ")
    base = ctype.replace("*", " ").replace("const", " ").split()
    assert len(base) == 1, ctype
    mapped = _C_BASE.get(base[0], base[0])
    if stars == 0:
        return mapped
    inner = ("*const " if is_const else "*mut ") + mapped
    return "*mut " * (stars - 1) + inner


def _split_decl(decl: str) -> tuple[str, str]:
    """`const float* attn_norm` -> (`const float*`, `attn_norm`)."""
    decl = " ".join(decl.replace("*", "* ").split())
    m = re.match(r"^(.*?)([A-Za-z_]\w*)$", decl)
    assert m, decl
    return m.group(1).strip(), m.group(2)


def header_functions() -> dict[str, tuple[str, list[str]]]:
    text = _strip_c_comments(HEADER.read_text())
    out = {}
    for m in re.finditer(r"WH_API\s+([^;(]*?)\b(wh_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        types = []
        if params and params != "void":
            for p in params.split(","):
                t, _ = _split_decl(p)
                types.append(c_type_to_rust(t))
        out[name] = (c_type_to_rust(ret), types)
    return out


def header_structs() -> dict[str, list[tuple[str, str]]]:
    text = _strip_c_comments(HEADER.read_text())
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        assert m.group(1) == m.group(3)
        fields = []
        for decl in m.group(2).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            arr = re.match(r"^(.*?)([A-Za-z_]\w*)\[(\w+)\]$", decl)
            if arr:
                fields.append((arr.group(2), f"[{c_type_to_rust(arr.group(1).strip())}; {arr.group(3)}]"))
                continue
            first, *rest = [d.strip() for d in decl.split(",")]
            t, name = _split_decl(first)
            fields.append((name, c_type_to_rust(t)))
            for extra in rest:  # `int a, b, c`
                fields.append((extra, c_type_to_rust(t)))
        out[m.group(1)] = fields
    return out


def header_constants() -> dict[str, int]:
    text = _strip_c_comments(HEADER.read_text())
    out = {}
    for body in re.findall(r"enum\s*\w*\s*\{(.*?)\}", text, flags=re.S):
        for m in re.finditer(r"(WH_\w+)\s*=\s*(\d+)", body):
            out[m.group(1)] = int(m.group(2))
    for m in re.finditer(r"#define\s+(WH_\w+)\s+(.+)", text):
        value = re.sub(r"\(\s*size_t\s*\)", "", m.group(2)).strip()
        if re.fullmatch(r"[\d\s()<>*+]+", value):
            out[m.group(1)] = int(eval(value))  # integer arithmetic only (checked above)
    return out


def _norm_rust_type(t: str) -> str:
    return " ".join(t.replace("*const", "*const ").replace("*mut", "*mut ").split())


def crate_functions() -> dict[str, tuple[str, list[str]]]:
    text = _strip_rust_comments(CRATE.read_text())
    blocks = re.findall(r'extern\s+"C"\s*\{(.*?)\n\}', text, flags=re.S)
    assert len(blocks) == 1, "one extern \"C\" block"
    out = {}
    for m in re.finditer(r"pub\s+fn\s+(wh_\w+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", blocks[0], flags=re.S):
        name, params, ret = m.group(1), m.group(2).strip(), (m.group(3) or "()").strip()
        types = []
        if params:
            for p in params.split(","):
                if not p.strip():
                    continue
                pname, ptype = p.split(":", 1)
                types.append(_norm_rust_type(ptype))
        assert name not in out, f"{name} declared twice"
        out[name] = (_norm_rust_type(ret), types)
    return out


def crate_structs() -> dict[str, list[tuple[str, str]]]:
    text = _strip_rust_comments(CRATE.read_text())
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*(?:#\[[^\]]*\]\s*)*pub\s+struct\s+(\w+)\s*\{(.*?)\}", text, flags=re.S):
        fields = []
        for f in m.group(2).split(","):
            f = " ".join(f.split())
            if not f:
                continue
            fm = re.match(r"^(?:pub\s+)?(?:r#)?(\w+)\s*:\s*(.+)$", f)
            assert fm, f
            fields.append((fm.group(1), _norm_rust_type(fm.group(2))))
        out[m.group(1)] = fields
    return out


def crate_constants() -> dict[str, int]:
    text = _strip_rust_comments(CRATE.read_text())
    out = {}
    for m in re.finditer(r"pub\s+const\s+(WH_\w+)\s*:\s*\w+\s*=\s*([^;]+);", text):
        value = m.group(2).strip()
        assert re.fullmatch(r"[\d\s()<>*+]+", value), value
        out[m.group(1)] = int(eval(value))  # integer arithmetic only (checked above)
    return out


def test_type_mapping():
    assert c_type_to_rust("const wh_weight*") == "*const wh_weight"
    assert c_type_to_rust("wh_gguf**") == "*mut *mut wh_gguf"
    assert c_type_to_rust("const void**") == "*mut *const c_void"
    assert c_type_to_rust("size_t") == "usize"
    assert _split_decl("const float* attn_norm") == ("const float*", "attn_norm")


def test_header_parse_is_complete():
    # every WH_API line of the header is one parsed function (nothing skipped)
    text = _strip_c_comments(HEADER.read_text())
    assert len(header_functions()) == text.count("WH_API ") - 1  # minus the #define
    assert len(header_functions()) >= 70


def test_every_header_function_is_declared_with_the_same_signature():
    hdr, crate = header_functions(), crate_functions()
    missing = sorted(set(hdr) - set(crate))
    extra = sorted(set(crate) - set(hdr))
    assert not missing, f"not in the crate: {missing}"
    assert not extra, f"in the crate but not the header: {extra}"
    for name, (ret, params) in hdr.items():
        c_ret, c_params = crate[name]
        assert c_ret == ret, f"{name}: returns {c_ret}, header {ret}"
        assert len(c_params) == len(params), f"{name}: {len(c_params)} arguments, header {len(params)}"
        for i, (a, b) in enumerate(zip(c_params, params)):
            assert a == b, f"{name} argument {i}: {a}, header {b}"


@pytest.mark.parametrize("name", sorted(header_structs()))
def test_struct_fields_match_in_order(name):
    crate = crate_structs()
    assert name in crate, f"struct {name} missing from the crate"
    assert crate[name] == header_structs()[name]


def test_opaque_handles_are_declared():
    text = CRATE.read_text()
    for t in ("wh_stream_t", "wh_event_t", "wh_graph_t"):
        assert re.search(rf"pub type {t} = \*mut \w+;", text), t
    crate = crate_structs()
    for t in ("wh_weight", "wh_gguf"):
        assert crate.get(t) == [("_private", "[u8; 0]")], t


def test_constants_match():
    hdr, crate = header_constants(), crate_constants()
    assert {"WH_OK", "WH_ERR_TYPE_MISMATCH", "WH_TYPE_Q6_K", "WH_GEMV_STREAM", "WH_GGUF_F64",
            "WH_GGUF_MAX_DIMS", "WH_LLAMA_DECODE_NOALLOC_MAX_BYTES"} <= set(hdr)
    for k, v in hdr.items():
        assert crate.get(k) == v, f"{k}: crate {crate.get(k)}, header {v}"
    assert set(crate) == set(hdr)


def test_planted_signature_mistake_is_caught(tmp_path, monkeypatch):
    # a swapped argument type in the crate must fail the signature check
    text = CRATE.read_text()
    bad = text.replace("pub fn wh_free(dptr: *mut c_void) -> c_int;", "pub fn wh_free(dptr: *const c_void) -> c_int;")
    assert bad != text
    p = tmp_path / "lib.rs"
    p.write_text(bad)
    monkeypatch.setattr(__import__(__name__), "CRATE", p)
    with pytest.raises(AssertionError, match="wh_free argument 0"):
        test_every_header_function_is_declared_with_the_same_signature()
