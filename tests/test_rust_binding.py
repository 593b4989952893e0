"""The Rust FFI crate (rust/janus-hip-sys, no cargo in this image) against the
C headers it binds: every function declared in include/*.h has an extern item
with the same name, parameter count, parameter types and return type under
the C-to-Rust type rules below; every status, dtype, flag and mode constant
has the header's value; janus_model_config has the header's fields, types and
order (the struct crosses the boundary by pointer, so a missing or reordered
field would shift every later offset)."""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
LIB_RS = ROOT / "rust" / "janus-hip-sys" / "src" / "lib.rs"
HEADERS = sorted((ROOT / "include").glob("*.h"))

SCALARS = {"int": "c_int", "uint32_t": "u32", "int32_t": "i32", "size_t": "usize", "float": "c_float",
           "uint16_t": "u16", "uint64_t": "u64", "char": "c_char", "void": "c_void"}


def _c_to_rust(ctype: str) -> str:
    t = " ".join(ctype.replace("*", " * ").split())
    stars = t.count("*")
    is_const = t.startswith("const ")
    base = t.replace("*", "").replace("const", "").strip()
    base = SCALARS.get(base, base)          # opaque / struct names keep their C name
    if stars == 0:
        return base
    if stars == 1:
        return ("*const " if is_const else "*mut ") + base
    assert stars == 2, ctype
    return "*mut *mut " + base


def _c_functions():
    out = {}
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"^\s*#.*$", "", text, flags=re.M)
        for decl in text.split(";"):
            m = re.search(r"([\w\s\*]+?)\b(janus_\w+)\s*\((.*)\)\s*$", decl.strip(), re.S)
            if not m or "typedef" in decl:
                continue
            ret, name, params = m.group(1), m.group(2), " ".join(m.group(3).split())
            args = []
            if params not in ("", "void"):
                for p in params.split(","):
                    pm = re.match(r"(.*?)(\w+)$", p.strip())
                    args.append(_c_to_rust(pm.group(1)))
            out[name] = (args, _c_to_rust(ret.replace("\n", " ")))
    return out


def _rust_functions():
    text = LIB_RS.read_text()
    block = text[text.index('unsafe extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (janus_\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, re.S):
        params = " ".join(m.group(2).split()).rstrip(",")
        args = [] if not params else [" ".join(p.split(":", 1)[1].split()) for p in params.split(",")]
        out[m.group(1)] = (args, (m.group(3) or "c_void").strip())
    return out


def _c_constants():
    vals = {}
    for h in HEADERS:
        text = h.read_text()
        for em in re.finditer(r"typedef enum \w+ \{(.*?)\}", text, re.S):
            for c in re.finditer(r"(JANUS_\w+)\s*=\s*(\d+)", em.group(1)):
                vals[c.group(1)] = int(c.group(2))
        for d in re.finditer(r"#define (JANUS_\w+)\s+\(?(0x[0-9a-fA-F]+|\d+)u?(?:\s*<<\s*(\d+))?\)?", text):
            if not d.group(1).endswith("_H"):
                vals[d.group(1)] = int(d.group(2), 0) << int(d.group(3) or 0)
    return vals


def test_every_header_function_has_a_matching_extern_item():
    c, rs = _c_functions(), _rust_functions()
    assert len(c) >= 50
    assert set(c) == set(rs), (sorted(set(c) - set(rs)), sorted(set(rs) - set(c)))
    for name, (args, ret) in c.items():
        rargs, rret = rs[name]
        assert rargs == args, (name, args, rargs)
        assert rret == ret, (name, ret, rret)


def test_constants_match_the_headers():
    want = _c_constants()
    got = {m.group(1): int(m.group(2), 0)
           for m in re.finditer(r"pub const (JANUS_\w+): \w+ = (0x[0-9a-fA-F]+|\d+);", LIB_RS.read_text())}
    assert len(want) >= 20
    assert got == want


def test_model_config_layout_matches_the_header():
    h = (ROOT / "include" / "janus_model.h").read_text()
    body = re.search(r"typedef struct janus_model_config \{(.*?)\} janus_model_config;", h, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    cfields = [(n, SCALARS[t]) for t, n in re.findall(r"\b(uint32_t|float|int)\s+(\w+)\s*;", body)]
    rs = LIB_RS.read_text()
    rbody = re.search(r"pub struct janus_model_config \{(.*?)\n\}", rs, re.S).group(1)
    rfields = re.findall(r"pub (\w+): (\w+),", rbody)
    assert len(cfields) == 13
    assert rfields == cfields
    assert "#[repr(C)]\n#[derive(Clone, Copy, Debug, Default)]\npub struct janus_model_config" in rs


def test_token_callback_type_matches_the_header():
    """janus_token_callback crosses the boundary as a nullable function
    pointer with the header's parameter and return types."""
    h = (ROOT / "include" / "janus_model.h").read_text()
    m = re.search(r"typedef (\w+) \(\*janus_token_callback\)\((.*?)\);", h, re.S)
    cargs = [_c_to_rust(re.match(r"(.*?)(\w+)$", p.strip()).group(1)) for p in m.group(2).split(",")]
    r = re.search(r"pub type janus_token_callback = Option<unsafe extern \"C\" fn\((.*?)\) -> (\w+)>;",
                  LIB_RS.read_text())
    rargs = [" ".join(p.split(":", 1)[1].split()) for p in r.group(1).split(",")]
    assert rargs == cargs
    assert r.group(2) == _c_to_rust(m.group(1))
