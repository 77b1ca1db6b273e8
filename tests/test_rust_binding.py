"""CPU check of the Rust binding (qmoe-rs_amd/rust/qmla-sys/src/lib.rs)
against the C header: cargo is not available on the build host, so the
crate cannot be compiled here; instead its `extern "C"` block and
`#[repr(C)]` structs are parsed and compared with include/qmla.h --
every entry point declared once, same argument names and order, argument
and return types that map one to one, struct fields in header order with
matching types, and the status / dtype constants."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qmla.h")
SYS_RS = os.path.join(ROOT, "qmoe-rs_amd", "rust", "qmla-sys", "src", "lib.rs")
BUILD_RS = os.path.join(ROOT, "qmoe-rs_amd", "rust", "qmla-sys", "build.rs")

_C_BASE = {"int32_t": "i32", "int": "c_int", "size_t": "usize", "double": "f64", "float": "f32",
           "uint64_t": "u64", "int64_t": "i64", "uint8_t": "u8", "uint16_t": "u16", "void": "c_void",
           "char": "c_char"}


def _strip_c_comments(t):
    return re.sub(r"/\*.*?\*/", "", t, flags=re.S)


def c_type(decl: str) -> str:
    """'const float *' -> '*const f32'; 'qmla_kv_cache **' -> '*mut *mut qmla_kv_cache'."""
    d = decl.strip()
    const = d.startswith("const ")
    if const:
        d = d[6:].strip()
    stars = d.count("*")
    base = _C_BASE.get(d.replace("*", "").strip(), d.replace("*", "").strip())
    out = base
    for i in range(stars):
        out = ("*const " if (i == 0 and const) else "*mut ") + out
    return out


def header_functions():
    t = _strip_c_comments(open(HEADER).read())
    funcs = {}
    for m in re.finditer(r"^QMLA_API\s+(.*?)\b(qmla_\w+)\s*\((.*?)\);", t, flags=re.S | re.M):
        ret, name, args = m.group(1), m.group(2), " ".join(m.group(3).split())
        params = []
        if args != "void":
            for a in args.split(","):
                mm = re.match(r"(.*?)(\w+)$", a.strip())
                params.append((mm.group(2), c_type(mm.group(1))))
        funcs[name] = (c_type(ret), params)
    return funcs


def header_structs():
    t = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"typedef struct \{(.*?)\}\s*(\w+);", t, flags=re.S):
        fields = []
        for line in m.group(1).split(";"):
            line = " ".join(line.split())
            if not line:
                continue
            mm = re.match(r"(.*?)(\w+(?:\s*,\s*\w+)*)$", line)
            ty = mm.group(1).strip()
            for name in mm.group(2).split(","):
                name = name.strip()
                stars = ty.count("*")
                fields.append((name, c_type(ty)))
            del stars
        out[m.group(2)] = fields
    return out


def _norm_rs(t: str) -> str:
    return " ".join(t.replace("*const", "*const ").replace("*mut", "*mut ").split())


def rust_functions():
    t = open(SYS_RS).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', t, flags=re.S).group(1)
    block = re.sub(r"//[^\n]*", "", block)
    funcs = {}
    for m in re.finditer(r"pub fn (qmla_\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        name, args, ret = m.group(1), " ".join(m.group(2).split()), m.group(3)
        params = []
        for a in filter(None, (x.strip() for x in args.split(","))):
            pn, ty = a.split(":", 1)
            params.append((pn.strip(), _norm_rs(ty)))
        assert name not in funcs, f"{name} declared twice"
        funcs[name] = (_norm_rs(ret) if ret else "c_void", params)
    return funcs


def rust_structs():
    t = open(SYS_RS).read()
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*(?:#\[derive[^\]]*\]\s*)?pub struct (\w+) \{(.*?)\}", t, flags=re.S):
        fields = []
        for line in m.group(2).split(","):
            line = line.strip()
            if line.startswith("pub "):
                pn, ty = line[4:].split(":", 1)
                fields.append((pn.strip(), _norm_rs(ty)))
        out[m.group(1)] = fields
    return out


def test_every_header_entry_point_is_bound_with_the_same_signature():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 46
    assert set(h) == set(r), f"missing in Rust: {set(h) - set(r)}; extra: {set(r) - set(h)}"
    for name, (ret, params) in h.items():
        rret, rparams = r[name]
        assert rret == ret, f"{name}: returns {rret}, header {ret}"
        assert [p for p, _ in rparams] == [p for p, _ in params], f"{name}: argument names/order differ"
        assert [t for _, t in rparams] == [t for _, t in params], f"{name}: argument types differ"


def test_repr_c_structs_match_the_header_field_order_and_types():
    h, r = header_structs(), rust_structs()
    for name in ("qmla_prefill_dims", "qmla_cache_desc", "qmla_decode_dims", "qmla_layer_config",
                 "qmla_moe_config"):
        assert name in h and name in r, name
        assert r[name] == h[name], f"{name}: Rust {r[name]} vs header {h[name]}"
    # opaque handles are declared as zero-sized repr(C) structs
    t = open(SYS_RS).read()
    for name in ("qmla_kv_cache", "qmla_layer"):
        assert re.search(rf"#\[repr\(C\)\]\s*pub struct {name} \{{\s*_private: \[u8; 0\],\s*\}}", t), name


def test_constants_match_the_header():
    ht = open(HEADER).read()
    rt = open(SYS_RS).read()
    for name, val in re.findall(r"\b(QMLA_(?:OK|ERR_\w+|F32|BF16))\s*=\s*(\d+)", ht):
        assert re.search(rf"pub const {name}: \w+ = {val};", rt), name
    assert re.search(r"#define QMLA_VERSION (\d+)", ht).group(1) in re.search(
        r"pub const QMLA_VERSION: c_int = (\d+);", rt).group(1)
    mib = int(re.search(r"#define QMLA_DECODE_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << 20\)", ht).group(1))
    assert f"pub const QMLA_DECODE_NOALLOC_SCRATCH_BYTES: usize = {mib} << 20;" in rt


def test_build_script_compiles_for_gfx950_and_links_the_runtime():
    b = open(BUILD_RS).read()
    mk = open(os.path.join(ROOT, "qmoe-rs_amd", "Makefile")).read()
    assert "--offload-arch=gfx950" in mk
    for lib in ("qmla", "amdhip64", "rocblas"):
        assert f"rustc-link-lib=dylib={lib}" in b
    assert 'Command::new("make")' in b
