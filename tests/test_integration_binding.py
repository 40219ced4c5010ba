"""The documented Rust binding for vasr-paged-attn against include/vpa.h (CPU).

The `extern "C"` block a maintainer would add to vasr-paged-attn must
declare every entry point of the C header with the same parameters, in the
same order, with the Rust type of each C type; a change of the ABI that the
documented binding does not follow fails here."""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

C_TO_RUST = {
    "int": "c_int", "int32_t": "i32", "int64_t": "i64", "uint32_t": "u32", "uint8_t": "u8",
    "size_t": "usize", "float": "f32", "char": "c_char", "void": "c_void",
}


def rust_type(c: str) -> str:
    c = " ".join(c.replace("*", " * ").split())
    const = c.startswith("const ")
    base = c[6:] if const else c
    stars = base.count("*")
    base = base.replace("*", "").strip()
    t = C_TO_RUST[base]
    for _ in range(stars):
        t = ("*const " if const else "*mut ") + t
    return t


def c_declarations():
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "vpa.h")).read(),
                  flags=re.S)
    text = "\n".join(l for l in text.splitlines()
                     if not l.lstrip().startswith("#") and "extern \"C\"" not in l)
    out = {}
    for chunk in text.replace("}", ";").split(";"):
        m = re.fullmatch(r"\s*([A-Za-z_][\w\s\*]*?)\b(vpa_\w+)\s*\(([^)]*)\)\s*", chunk)
        if m is None:
            continue
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        params = []
        if args and args != "void":
            for a in args.split(","):
                a = " ".join(a.split())
                mm = re.match(r"(.*?)([A-Za-z_]\w*)$", a)
                params.append((mm.group(2), rust_type(mm.group(1).strip())))
        out[name] = (rust_type(ret), params)
    return out


def rust_declarations():
    md = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = md[md.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    out = {}
    for m in re.finditer(r"pub fn (vpa_\w+)\((.*?)\)\s*(?:->\s*([^;]+))?;", block, re.S):
        params = []
        for a in m.group(2).split(","):
            if a.strip():
                n, t = a.split(":", 1)
                params.append((n.strip(), " ".join(t.split())))
        out[m.group(1)] = ((m.group(3) or "()").strip(), params)
    return out


def test_rust_binding_declares_every_entry_point_of_vpa_h():
    c, rs = c_declarations(), rust_declarations()
    assert len(c) >= 17
    assert sorted(rs) == sorted(c)
    for name, (ret, params) in c.items():
        assert rs[name][0] == ret, name
        assert rs[name][1] == params, name
