"""Signatures of the C ABI header and of the Rust FFI block that
INTEGRATION.md gives a maintainer, both reduced to Rust types, so a test can
compare them declaration by declaration (tests/test_host.py)."""
import re

PRIM = {"uint8_t": "u8", "uint16_t": "u16", "uint32_t": "u32", "uint64_t": "u64", "int8_t": "i8",
        "int32_t": "i32", "int64_t": "i64", "int": "c_int", "float": "f32", "double": "f64",
        "size_t": "usize", "char": "c_char", "void": "c_void"}


def strip_comments(t):
    return re.sub(r"/\*.*?\*/", "", t, flags=re.S)


def c_type_to_rust(decl):
    """'const fbh_shape *shape' -> ('shape', '*const fbh_shape')"""
    decl = decl.strip()
    arr = re.search(r"\[(\d*)\]\s*$", decl)
    if arr:
        decl = decl[:arr.start()].strip()
    m = re.match(r"^(.*?)(\w+)$", decl)
    ty, name = m.group(1).strip(), m.group(2)
    const = ty.startswith("const ")
    if const:
        ty = ty[6:].strip()
    stars = ty.count("*")
    base = ty.replace("*", "").strip()
    base = PRIM.get(base, base)
    if arr:
        stars += 1
    if stars == 0:
        return name, base
    out = base
    for i in range(stars):
        innermost = i == 0
        out = ("*const " if (innermost and const) else "*mut ") + out
    return name, out


def header_functions(text):
    text = strip_comments(text)
    funcs = {}
    for m in re.finditer(r"^\s*(int|size_t|uint64_t|uint32_t|double|void|float)\s+(fb[ht]_\w+)\s*\(([^;]*?)\)\s*;",
                         text, flags=re.S | re.M):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        args = [a.strip() for a in args.replace("\n", " ").split(",") if a.strip() and a.strip() != "void"]
        funcs[name] = (PRIM.get(ret, ret), [c_type_to_rust(a) for a in args])
    return funcs


def header_structs(text):
    text = strip_comments(text)
    out = {}
    for m in re.finditer(r"typedef\s+struct\s*(\w*)\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        body, name = m.group(2), m.group(3)
        fields = []
        for line in body.split(";"):
            line = " ".join(line.split())
            if not line:
                continue
            # 'uint32_t feat, bin' style
            mm = re.match(r"^(const\s+)?([\w]+)\s*(\**)\s*(.*)$", line)
            const, base, stars, names = mm.groups()
            for nm in names.split(","):
                nm = nm.strip()
                st = stars + "".join("*" for _ in range(nm.count("*")))
                nm = nm.replace("*", "").strip()
                arr = re.search(r"\[(\d+)\]$", nm)
                n = nm[:arr.start()] if arr else nm
                ty = PRIM.get(base, base)
                for i in range(len(st)):
                    ty = ("*const " if (i == 0 and const) else "*mut ") + ty
                if arr:
                    ty = f"[{ty}; {arr.group(1)}]"
                fields.append((n, ty))
        out[name] = fields
    return out


def rust_block(markdown: str) -> str:
    """The ```rust block of INTEGRATION.md that holds `extern "C"`."""
    for m in re.finditer(r"```rust\n(.*?)```", markdown, flags=re.S):
        if 'extern "C"' in m.group(1):
            return m.group(1)
    raise ValueError("no rust extern block")


def _norm(ty: str) -> str:
    return " ".join(ty.replace("std::os::raw::", "").split())


def rust_functions(block: str):
    body = block[block.index('extern "C"'):]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    body = re.sub(r"//[^\n]*", "", body)
    out = {}
    for m in re.finditer(r"pub fn (\w+)\((.*?)\)\s*(?:->\s*([\w:]+))?\s*;", body, flags=re.S):
        name, args, ret = m.group(1), m.group(2), m.group(3) or "()"
        parts = [a.strip() for a in args.split(",") if a.strip()]
        out[name] = (_norm(ret), [(a.split(":", 1)[0].strip(), _norm(a.split(":", 1)[1]))
                                  for a in parts])
    return out


def rust_structs(block: str):
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub struct (\w+)\s*\{(.*?)\}", block, flags=re.S):
        name, body = m.group(1), m.group(2)
        fields = []
        for f in re.finditer(r"pub (\w+):\s*([^,]+?)\s*(?:,|$)", body.strip() + ","):
            fields.append((f.group(1), _norm(f.group(2))))
        out[name] = fields
    return out
