"""rust/nf4_hip.rs, the `extern "C"` module a maintainer adds to the Rust
crates, against include/nf4stream.h: the same functions with the same
argument types and names, return types, status constants and struct layouts.
CPU only; the image has no Rust toolchain, so this is a text check of the two
declarations against one C-to-Rust type mapping."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nf4stream.h")
RUST = os.path.join(ROOT, "rust", "nf4_hip.rs")

BASE = {"int32_t": "i32", "int64_t": "i64", "uint32_t": "u32", "uint16_t": "u16",
        "uint8_t": "u8", "float": "f32", "char": "c_char", "void": "c_void",
        "nf4s_tensor": "Nf4sTensor", "nf4s_param_info": "Nf4sParamInfo",
        "nf4s_dbuf": "Nf4sDbuf", "nf4s_loader": "Nf4sLoader",
        "nf4s_ready_layer": "Nf4sReadyLayer", "nf4s_blob_entry": "Nf4sBlobEntry",
        "nf4s_residency": "Nf4sResidency"}


def c_to_rust(ctype: str) -> str:
    """`const uint16_t *const *` -> `*const *const u16`: each '*' wraps the
    type so far in a pointer whose Rust mutability is the pointee's constness;
    a `const` after a '*' makes that pointer itself const."""
    toks = re.findall(r"\*|[A-Za-z_][A-Za-z0-9_]*", ctype)
    const = False
    if toks[0] == "const":
        const, toks = True, toks[1:]
    ty = BASE[toks[0]]
    for t in toks[1:]:
        if t == "*":
            ty = ("*const " if const else "*mut ") + ty
            const = False
        elif t == "const":
            const = True
        else:
            raise ValueError(ctype)
    return ty


def c_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"(int32_t|int64_t|const char \*)\s*(nf4s_\w+)\s*\(([^;]*?)\)\s*;",
                         text, re.S):
        ret, name, params = m.group(1), m.group(2), " ".join(m.group(3).split())
        args = []
        if params != "void":
            for p in params.split(","):
                p = p.strip()
                pm = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)$", p)
                args.append((pm.group(2), c_to_rust(pm.group(1).strip())))
        out[name] = (c_to_rust(ret.replace(" ", " ")), args)
    return out


def rust_functions():
    text = open(RUST).read()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    out = {}
    for m in re.finditer(r"pub fn (nf4s_\w+)\((.*?)\)\s*(?:->\s*([^;]+))?;", block, re.S):
        name, params, ret = m.group(1), " ".join(m.group(2).split()), m.group(3)
        args = []
        if params.strip():
            for p in params.split(","):
                p = p.strip()
                if not p:
                    continue
                a, t = p.split(":", 1)
                args.append((a.strip(), " ".join(t.split())))
        out[name] = (" ".join(ret.split()) if ret else "()", args)
    return out


def test_every_header_function_is_declared_alike():
    c, r = c_functions(), rust_functions()
    assert len(c) == len(set(re.findall(r"\b(nf4s_[a-z0-9_]+)\s*\(", open(HEADER).read())))
    assert sorted(c) == sorted(r)
    for name, (ret, args) in c.items():
        assert r[name][0] == ret, (name, r[name][0], ret)
        assert r[name][1] == args, (name, r[name][1], args)


def test_type_mapping_examples():
    assert c_to_rust("const uint16_t *const *") == "*const *const u16"
    assert c_to_rust("uint16_t *const *") == "*const *mut u16"
    assert c_to_rust("void **") == "*mut *mut c_void"
    assert c_to_rust("const uint8_t **") == "*mut *const u8"
    assert c_to_rust("const char *const *") == "*const *const c_char"


def test_status_constants_and_version():
    h = open(HEADER).read()
    rs = open(RUST).read()
    consts = dict(re.findall(r"(NF4S_\w+)\s*=\s*(\d+)", h))
    assert len(consts) == 19  # 13 status codes, 6 precisions
    for k, v in consts.items():
        assert re.search(rf"pub const {k}: i32 = {v};", rs), k
    ver = re.search(r"#define NF4S_ABI_VERSION (\d+)", h).group(1)
    assert re.search(rf"pub const NF4S_ABI_VERSION: i32 = {ver};", rs)


def _c_struct(name):
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\}" % name, text, re.S).group(1)
    fields = []
    for line in body.split(";"):
        line = " ".join(line.split())
        if not line:
            continue
        m = re.match(r"(.*?)([A-Za-z_]\w*)(\[(\d+)\])?$", line)
        ty = c_to_rust(m.group(1).strip())
        if m.group(4):
            ty = f"[{ty}; {m.group(4)}]"
        fields.append((m.group(2), ty))
    return fields


def _rust_struct(name):
    text = open(RUST).read()
    body = re.search(r"pub struct %s \{(.*?)\}" % name, text, re.S).group(1)
    return [(a.strip(), " ".join(t.split())) for a, t in
            re.findall(r"pub (\w+):\s*([^,]+),", body)]


def test_struct_layouts_match():
    for c, rs in [("nf4s_tensor", "Nf4sTensor"), ("nf4s_param_info", "Nf4sParamInfo"),
                  ("nf4s_ready_layer", "Nf4sReadyLayer"), ("nf4s_blob_entry", "Nf4sBlobEntry")]:
        assert _c_struct(c) == _rust_struct(rs), c
