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


# ---- the candle drop-ins against the reference's public API -------------
# The reference's signatures, written out from qmoe-rs src/model.rs and
# src/attention_kernel.rs (whitespace-normalised): the engine calls these,
# so the drop-ins must accept the same calls.
MODEL_RS = os.path.join(ROOT, "qmoe-rs_amd", "rust", "qmla", "src", "model.rs")
KERNEL_RS = os.path.join(ROOT, "qmoe-rs_amd", "rust", "qmla", "src", "attention_kernel.rs")
LIB_RS = os.path.join(ROOT, "qmoe-rs_amd", "rust", "qmla", "src", "lib.rs")

REF_METHODS = {  # src/model.rs:125, :193, :256
    "new": "(vb: VarBuilder, config: &ModelConfig) -> Result<Self>",
    "forward_prefill": "(&self, xs: &Tensor) -> Result<(Tensor, KVCache)>",
    "forward_with_cache": "(&self, xs: &Tensor, cache: &mut KVCache) -> Result<Tensor>",
}
REF_FIELDS = [  # pub fields of MlaAttention, src/model.rs:108-122
    ("q_proj", "candle_nn::Linear"), ("kv_a_proj_with_mqa", "candle_nn::Linear"),
    ("kv_a_layernorm", "candle_nn::LayerNorm"), ("kv_b_proj", "candle_nn::Linear"),
    ("o_proj", "candle_nn::Linear"), ("num_heads", "usize"), ("num_kv_heads", "usize"),
    ("qk_nope_head_dim", "usize"), ("qk_rope_head_dim", "usize"), ("v_head_dim", "usize"),
    ("kv_lora_rank", "usize"), ("rope_mscale", "f64"), ("softmax_scale", "f64"),
]
REF_CONFIG_FIELDS = ["hidden_size", "num_attention_heads", "num_key_value_heads", "qk_nope_head_dim",
                     "qk_rope_head_dim", "v_head_dim", "kv_lora_rank"]  # src/model.rs:8-20
REF_KERNELS = {  # src/attention_kernel.rs:34, :64, :110
    "eager_prefill_attn": "(q: &Tensor, k: &Tensor, v: &Tensor, scale: f64, causal: bool) -> Result<Tensor>",
    "fused_prefill_attn": "(q_nope: &Tensor, q_rope: &Tensor, k: &Tensor, k_rope: &Tensor, v: &Tensor, "
                          "scale: f64, causal: bool) -> Result<Tensor>",
    "reference_eager_attn": "(q: &Tensor, k: &Tensor, v: &Tensor, scale: f64, causal: bool) -> Result<Tensor>",
}


def _pub_fns(text, impl_of=None):
    """{name: normalised '(args) -> ret'} of the `pub fn`s (inside `impl impl_of` if given)."""
    if impl_of:
        m = re.search(rf"\nimpl {impl_of} \{{\n(.*?)\n\}}\n", text, flags=re.S)
        text = m.group(1)
    out = {}
    for m in re.finditer(r"pub fn (\w+)\s*(<[^>]*>)?\s*(\(.*?\))\s*->\s*([^{]+?)\s*\{", text, flags=re.S):
        args = " ".join(m.group(3).split()).replace("( ", "(").replace(", )", ")")
        out[m.group(1)] = (m.group(2) or "", f"{args} -> {' '.join(m.group(4).split())}")
    return out


def test_mla_attention_keeps_the_reference_constructor_and_methods():
    t = open(MODEL_RS).read()
    fns = _pub_fns(t, "MlaAttention")
    for name in ("forward_prefill", "forward_with_cache"):
        assert fns[name][1] == REF_METHODS[name], (name, fns[name])
    # new(vb, config): the engine's &ModelConfig is accepted through MlaConfig
    generics, sig = fns["new"]
    assert generics.replace(" ", "") == "<C:MlaConfig+?Sized>", generics
    assert sig.replace("&C", "&ModelConfig") == REF_METHODS["new"], sig
    # the reference's VarBuilder paths and module constructors, :126-146
    for path, ctor in (("q_proj", "linear"), ("kv_a_proj_with_mqa", "linear"),
                       ("kv_a_layernorm", "layer_norm"), ("kv_b_proj", "linear"), ("o_proj", "linear")):
        assert re.search(rf"candle_nn::{ctor}\([^;]*vb\.pp\(\"{path}\"\)\)", t), path
    assert "layer_norm(r, 1e-6," in t  # LayerNorm eps 1e-6, :136


def test_mla_attention_keeps_the_reference_pub_fields():
    t = open(MODEL_RS).read()
    body = re.search(r"pub struct MlaAttention \{(.*?)\n\}", t, flags=re.S).group(1)
    fields = re.findall(r"^\s*pub (\w+): ([\w:]+),", body, flags=re.M)
    got = dict(fields)
    for name, ty in REF_FIELDS:
        assert got.get(name) == ty, (name, got.get(name))
    # the field order of the reference comes first
    assert [n for n, _ in fields[:len(REF_FIELDS)]] == [n for n, _ in REF_FIELDS]


def test_config_macro_reads_the_reference_model_config_fields():
    t = open(MODEL_RS).read()
    mac = re.search(r"macro_rules! impl_mla_config \{(.*?)\n\}", t, flags=re.S).group(1)
    trait = re.search(r"pub trait MlaConfig \{(.*?)\n\}", t, flags=re.S).group(1)
    for f in REF_CONFIG_FIELDS:
        assert f"fn {f}(&self) -> usize" in trait, f
        assert re.search(rf"fn {f}\(&self\) -> usize \{{ self\.{f} \}}", mac), f


def test_kv_cache_is_clone_and_reads_the_reference_tensors():
    t = open(MODEL_RS).read()
    assert re.search(r"impl Clone for KVCache \{", t)
    fns = _pub_fns(t, "KVCache")
    for name in ("k", "v", "k_rope"):
        assert fns[name][1] == "(&self, layer: &MlaAttention) -> Result<Tensor>", (name, fns[name])
    assert "empty" in fns and "append" not in fns and "new" not in fns


def test_attention_kernel_drop_in_keeps_the_reference_signatures():
    fns = _pub_fns(open(KERNEL_RS).read())
    for name, sig in REF_KERNELS.items():
        assert fns[name][1] == sig, (name, fns[name])


def test_safe_wrappers_check_sizes_before_calling_c():
    """Every safe wrapper that hands caller slices or buffers to C checks
    their sizes first (a short one would be read or written past its end)."""
    t = open(LIB_RS).read()
    wanted = {"MlaAttention": ["new", "forward_with_cache", "forward_prefill", "materialise"],
              "KVCache": ["gather", "append", "set_lengths", "reserve"],
              "PackedQMoETensor": ["from_bytes", "forward"],
              "QMoELayer": ["new", "forward"],
              None: ["fused_prefill_attn", "decode_absorbed"]}
    for owner, names in wanted.items():
        scope = t
        if owner:
            scope = re.search(rf"\nimpl {owner} \{{\n(.*?)\n\}}\n", t, flags=re.S).group(1) + "\n"
        for name in names:
            end = r"\n    \}\n" if owner else r"\n\}\n"
            m = re.search(rf"pub fn {name}\b.*?\{{(.*?){end}", scope, flags=re.S)
            body = m.group(1)
            calls = [c for c in (body.find("unsafe"), body.find("from_slice(")) if c >= 0]
            first_unsafe = min(calls)
            checks = [body.find(k) for k in ("check_len(", "check_bytes(", "check_opt_len(",
                                              "self.check_io(", "shape_err(")]
            checks = [c for c in checks if c >= 0]
            assert checks and min(checks) < first_unsafe, f"{owner}::{name} calls C before checking sizes"
