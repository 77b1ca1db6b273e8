"""CPU checks of the C ABI boundary: the library loads, exports exactly what
include/qmla.h declares, and validates arguments before touching a device.
No compute call is made here (there is no GPU on the build host)."""
import ctypes as C
import os
import re
import subprocess

import pytest

import qmla

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qmla.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"QMLA_API\s+[\w\s\*]*?\b(qmla_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = header_symbols()
    for required in ("qmla_fused_prefill_attn", "qmla_reference_eager_attn", "qmla_eager_prefill_attn",
                     "qmla_cache_create", "qmla_cache_append", "qmla_cache_clone", "qmla_cache_lengths",
                     "qmla_decode_absorbed", "qmla_decode_workspace_bytes", "qmla_layer_forward_with_cache",
                     "qmla_layer_forward_prefill", "qmla_last_error"):
        assert required in syms


def test_library_exports_every_declared_symbol():
    if not os.path.exists(qmla.LIB_PATH):
        pytest.fail("libqmla.so is not built (run __graft_entry__.build())")
    out = subprocess.run(["nm", "-D", "--defined-only", qmla.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (qmla_\w+)$", out, re.M))
    declared = set(header_symbols())
    assert declared - exported == set(), f"declared but not exported: {declared - exported}"
    assert exported - declared == set(), f"exported but not declared: {exported - declared}"
    # and the Python binding knows every one of them
    assert declared == set(qmla.SIGNATURES)


def test_library_loads_and_reports_errors_without_a_device():
    L = qmla.lib()
    assert L.qmla_version() == 100
    assert L.qmla_status_string(6) == b"QMLA_ERR_CAPACITY"
    # argument validation happens before any HIP call
    assert L.qmla_fused_prefill_attn(None, 0, None, None, None, None, None, 1.0, 1, None, None) == 1
    assert b"dims is NULL" in L.qmla_last_error()
    dims = qmla.PrefillDims(1, 2, 4, 4, 16, 8, 16, 3, 0)  # k_rope_heads 3 is neither 1 nor heads
    st = L.qmla_fused_prefill_attn(C.byref(dims), 0, 1, 1, 1, 1, 1, 1.0, 1, 1, None)
    assert st == 2 and b"k_rope_heads" in L.qmla_last_error()
    dims = qmla.PrefillDims(1, 2, 4, 4, 16, 8, 16, 1, -3)
    assert L.qmla_fused_prefill_attn(C.byref(dims), 0, 1, 1, 1, 1, 1, 1.0, 1, 1, None) == 2
    dims = qmla.PrefillDims(1, 2, 4, 4, 16, 8, 16, 1, 0)
    assert L.qmla_fused_prefill_attn(C.byref(dims), 7, 1, 1, 1, 1, 1, 1.0, 1, 1, None) == 1
    assert L.qmla_fused_prefill_attn(C.byref(dims), 0, 1, 1, 1, 1, 1, float("nan"), 1, 1, None) == 1
    assert L.qmla_cache_create(0, None, 512, 64, 1, None) == 1
    h = C.c_void_p()
    caps = (C.c_int32 * 2)(4, 4)
    assert L.qmla_cache_create(2, caps, 500, 64, 1, C.byref(h)) == 3  # 564 % 8 != 0
    assert L.qmla_decode_absorbed(None, None, 0, None, None, 1.0, None, None, None, 0, None) == 1


def test_oracle_library_builds_and_loads():
    import oracle
    oracle.build(force=False)
    assert oracle.lib().orc_tile_size(2049) == 16


def test_packed_and_moe_argument_checks_without_a_device():
    """qmla_packed_forward / qmla_moe_forward validate sizes on the host and
    report their workspace (none for the packed GEMV) without a device."""
    L = qmla.lib()
    n = C.c_size_t(123)
    assert L.qmla_packed_forward_workspace_bytes(64, 2048, 16, C.byref(n)) == 0 and n.value == 0
    assert L.qmla_packed_forward_workspace_bytes(64, -4, 16, C.byref(n)) == 2
    assert L.qmla_packed_forward_workspace_bytes(64, (1 << 20) + 4, 1, C.byref(n)) == 3
    cfg = qmla.MoEConfig(32, 4, 2048, 1408)
    assert L.qmla_moe_workspace_bytes(C.byref(cfg), 16, C.byref(n)) == 0
    # routing, bins, h [64, 1408] and y [64, 2048] in f32 at least
    assert n.value >= 4 * 64 * (1408 + 2048)
    assert L.qmla_moe_workspace_bytes(C.byref(qmla.MoEConfig(4, 5, 64, 64)), 2, C.byref(n)) == 2
    assert b"top_k" in L.qmla_last_error()
    assert L.qmla_moe_workspace_bytes(C.byref(qmla.MoEConfig(5000, 2, 64, 64)), 2, C.byref(n)) == 3
    assert L.qmla_moe_workspace_bytes(None, 2, C.byref(n)) == 1
    # a zero-length call is a no-op that needs no pointers
    assert L.qmla_moe_forward(C.byref(cfg), None, 0, *([None] * 11), 0, None) == 0


def test_layer_default_scales_match_the_reference_constructor():
    """qmla_layer_default_scales restates MlaAttention::new's YaRN scales
    (src/model.rs:160-173): rope_mscale = mscale(40, 1) / mscale(40, 0.707)
    and softmax_scale = (dn + dr)^-1/2 * mscale(40, 0.707)^2, against the
    closed-form constants (ln 40 = 3.6888794541139363)."""
    L = qmla.lib()
    for dn, dr, want in ((128, 64, 0.1147213868), (32, 16, 0.2294427736)):
        cfg = qmla.LayerConfig(2048, 16, dn, dr, 128, 512, 0.0, 0.0, 0.0)
        assert L.qmla_layer_default_scales(C.byref(cfg)) == 0
        assert abs(cfg.rope_mscale - 1.0857263992) < 1e-9
        assert abs(cfg.softmax_scale - want) < 1e-9
        assert cfg.ln_eps == 1e-6
    m = 0.1 * 0.707 * 3.6888794541139363 + 1.0
    assert abs(m - 1.2608037767) < 1e-9
    assert abs((0.1 * 3.6888794541139363 + 1.0) / m - 1.0857263992) < 1e-9
    assert L.qmla_layer_default_scales(None) == 1


def test_materialise_and_layer_calls_validate_without_a_device():
    L = qmla.lib()
    n = C.c_size_t()
    assert L.qmla_cache_materialise_workspace_bytes(None, None, 0, 1, C.byref(n)) == 1
    assert L.qmla_cache_materialise(None, None, 0, 1, None, None, None, None, 0, None) == 1
    assert L.qmla_layer_forward_with_cache(None, None, 1, 1, None, None, None, 0, None) == 1
    assert L.qmla_layer_set_projection_dtype(None, qmla.BF16) == 1
