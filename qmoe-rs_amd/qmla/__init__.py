"""Python binding of libqmla.so, the MI355X MLA attention library.

A thin ctypes layer over the C ABI declared in include/qmla.h.  It mirrors
the reference's interface for this path (qmoe-rs src/attention_kernel.rs and
the KVCache / MlaAttention API of src/model.rs) with numpy arrays on the host
side and DeviceBuffer objects for HBM-resident tensors.  There is no CPU
fallback: if libqmla.so is missing or no GPU is present, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libqmla.so")

F32, BF16 = 0, 1
_DT = {F32: np.float32, BF16: np.uint16}

STATUS = {0: "QMLA_OK", 1: "QMLA_ERR_INVALID_ARG", 2: "QMLA_ERR_SHAPE", 3: "QMLA_ERR_UNSUPPORTED",
          4: "QMLA_ERR_HIP", 5: "QMLA_ERR_OOM", 6: "QMLA_ERR_CAPACITY", 7: "QMLA_ERR_WORKSPACE"}


class QmlaError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS.get(status, status)}: {msg}")
        self.status = status


def build(force: bool = True) -> str:
    """Compile libqmla.so in-tree with hipcc for gfx950."""
    jobs = str(min(8, os.cpu_count() or 1))
    args = ["make", "-C", PKG_DIR, "-j", jobs]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)
    return LIB_PATH


# ------------------------------------------------------------ ctypes types

class PrefillDims(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("batch", "heads", "seq_q", "seq_k", "qk_nope", "qk_rope",
                                         "v_dim", "k_rope_heads", "q_offset")]


class DecodeDims(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("batch", "rows", "kv_lora_rank", "rope_dim")]


class CacheDesc(C.Structure):
    _fields_ = [("num_seqs", C.c_int32), ("kv_lora_rank", C.c_int32), ("rope_dim", C.c_int32),
                ("dtype", C.c_int), ("row_elems", C.c_int64), ("total_rows", C.c_int64),
                ("rows", C.c_void_p), ("offsets", C.c_void_p), ("lengths", C.c_void_p),
                ("capacity", C.c_void_p), ("pages", C.c_void_p), ("page_rows", C.c_int32),
                ("table_width", C.c_int32), ("contiguous", C.c_int32), ("reserved", C.c_int32)]


class LayerConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("hidden", "heads", "qk_nope", "qk_rope", "v_dim",
                                         "kv_lora_rank")] + [
        ("rope_mscale", C.c_double), ("softmax_scale", C.c_double), ("ln_eps", C.c_double)]


class MoEConfig(C.Structure):
    """MoEConfig (src/moe.rs:5-11)."""
    _fields_ = [(n, C.c_int32) for n in ("num_experts", "top_k", "hidden_dim", "intermediate_dim")]


# Every symbol include/qmla.h declares, with its ctypes signature.
_vp, _i32, _sz, _d, _u64 = C.c_void_p, C.c_int32, C.c_size_t, C.c_double, C.c_uint64
_st = C.c_int
SIGNATURES = {
    "qmla_version": (C.c_int, []),
    "qmla_last_error": (C.c_char_p, []),
    "qmla_status_string": (C.c_char_p, [_st]),
    "qmla_device_info": (_st, [C.POINTER(C.c_int), C.POINTER(C.c_int), C.c_char_p, _sz]),
    "qmla_buffer_alloc": (_st, [_sz, C.POINTER(_vp)]),
    "qmla_buffer_free": (_st, [_vp]),
    "qmla_memcpy_h2d": (_st, [_vp, _vp, _sz, _vp]),
    "qmla_memcpy_d2h": (_st, [_vp, _vp, _sz, _vp]),
    "qmla_memcpy_d2d": (_st, [_vp, _vp, _sz, _vp]),
    "qmla_memset_zero": (_st, [_vp, _sz, _vp]),
    "qmla_stream_create": (_st, [C.POINTER(_vp)]),
    "qmla_stream_destroy": (_st, [_vp]),
    "qmla_stream_synchronize": (_st, [_vp]),
    "qmla_f32_to_bf16": (_st, [_vp, _vp, _sz, _vp]),
    "qmla_fill_normal_f32": (_st, [_vp, _sz, _u64, C.c_float, C.c_float, _vp]),
    "qmla_fused_prefill_attn": (_st, [C.POINTER(PrefillDims), _st, _vp, _vp, _vp, _vp, _vp, _d, C.c_int,
                                      _vp, _vp]),
    "qmla_reference_eager_attn": (_st, [_i32] * 5 + [_st, _vp, _vp, _vp, _d, C.c_int, _vp, _vp]),
    "qmla_eager_prefill_attn": (_st, [_i32] * 5 + [_st, _vp, _vp, _vp, _d, C.c_int, _vp, _vp]),
    "qmla_cache_create": (_st, [_i32, C.POINTER(_i32), _i32, _i32, _st, C.POINTER(_vp)]),
    "qmla_cache_create_paged": (_st, [_i32, C.POINTER(_i32), C.c_int64, C.c_int64, _i32, _i32, _i32, _st,
                                      C.POINTER(_vp)]),
    "qmla_cache_destroy": (_st, [_vp]),
    "qmla_cache_clone": (_st, [_vp, C.POINTER(_vp), _vp]),
    "qmla_cache_append": (_st, [_vp, _vp, _st, _i32, _i32, _vp]),
    "qmla_cache_append_seq": (_st, [_vp, _i32, _vp, _st, _i32, _vp]),
    "qmla_cache_set_lengths": (_st, [_vp, C.POINTER(_i32), _vp]),
    "qmla_cache_lengths": (_st, [_vp, C.POINTER(_i32)]),
    "qmla_cache_describe": (_st, [_vp, C.POINTER(CacheDesc)]),
    "qmla_cache_gather": (_st, [_vp, _i32, _i32, _i32, _vp, _vp]),
    "qmla_cache_reserve": (_st, [_vp, C.POINTER(_i32), _vp]),
    "qmla_cache_set_growth": (_st, [_vp, _i32]),
    "qmla_cache_capacity": (_st, [_vp, C.POINTER(_i32)]),
    "qmla_cache_reserve_pool": (_st, [_vp, C.c_int64]),
    "qmla_cache_trim": (_st, [_vp, _i32, _i32, _vp]),
    "qmla_cache_pool_info": (_st, [_vp, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "qmla_decode_workspace_bytes": (_st, [C.POINTER(DecodeDims), _vp, C.POINTER(_sz)]),
    "qmla_decode_workspace_bytes_splits": (_st, [C.POINTER(DecodeDims), _vp, _i32, C.POINTER(_sz)]),
    "qmla_decode_absorbed": (_st, [C.POINTER(DecodeDims), _vp, _st, _vp, _vp, _d, _vp, _vp, _vp, _sz, _vp]),
    "qmla_decode_absorbed_splits": (_st, [C.POINTER(DecodeDims), _vp, _st, _vp, _vp, _d, _vp, _vp, _i32,
                                          _vp, _sz, _vp]),
    "qmla_decode_absorbed_noalloc": (_st, [C.POINTER(DecodeDims), _vp, _st, _vp, _vp, _d, _vp, _vp, _vp]),
    "qmla_layer_default_scales": (_st, [C.POINTER(LayerConfig)]),
    "qmla_layer_create": (_st, [C.POINTER(LayerConfig)] + [_vp] * 10 + [C.POINTER(_vp)]),
    "qmla_layer_destroy": (_st, [_vp]),
    "qmla_layer_set_projection_dtype": (_st, [_vp, _st]),
    "qmla_layer_workspace_bytes": (_st, [_vp, _vp, _i32, _i32, C.POINTER(_sz)]),
    "qmla_layer_prefill_workspace_bytes": (_st, [_vp, _vp, _i32, _i32, C.POINTER(_sz)]),
    "qmla_layer_forward_with_cache": (_st, [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "qmla_layer_forward_prefill": (_st, [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "qmla_cache_materialise_workspace_bytes": (_st, [_vp, _vp, _i32, _i32, C.POINTER(_sz)]),
    "qmla_cache_materialise": (_st, [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _sz, _vp]),
    "qmla_packed_forward_workspace_bytes": (_st, [_i32, _i32, _i32, C.POINTER(_sz)]),
    "qmla_packed_forward": (_st, [_vp, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _sz, _vp]),
    "qmla_moe_workspace_bytes": (_st, [C.POINTER(MoEConfig), _i32, C.POINTER(_sz)]),
    "qmla_moe_forward": (_st, [C.POINTER(MoEConfig), _vp, _i32] + [_vp] * 7 + [_vp, _vp, _vp, _vp, _sz, _vp]),
}

_lib = None


def lib():
    """Load libqmla.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run qmla.build() (make -C qmoe-rs_amd)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int):
    if status != 0:
        msg = lib().qmla_last_error().decode(errors="replace")
        raise QmlaError(status, msg)


def device_info():
    dev, cus = C.c_int(), C.c_int()
    name = C.create_string_buffer(64)
    check(lib().qmla_device_info(C.byref(dev), C.byref(cus), name, 64))
    return dev.value, cus.value, name.value.decode()


# ------------------------------------------------------------ device memory

class Stream:
    def __init__(self):
        h = C.c_void_p()
        check(lib().qmla_stream_create(C.byref(h)))
        self.handle = h.value

    def sync(self):
        check(lib().qmla_stream_synchronize(self.handle))

    def close(self):
        if self.handle:
            lib().qmla_stream_destroy(self.handle)
            self.handle = None


class DeviceBuffer:
    """An HBM allocation owned by Python (qmla_buffer_alloc / free)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().qmla_buffer_alloc(max(self.nbytes, 1), C.byref(p)))
        self.ptr = p.value

    @staticmethod
    def from_numpy(a: np.ndarray, stream=None) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = DeviceBuffer(a.nbytes)
        if a.nbytes:
            check(lib().qmla_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes, _sh(stream)))
            check(lib().qmla_stream_synchronize(_sh(stream)))
        return b

    def to_numpy(self, dtype, shape, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        if out.nbytes:
            check(lib().qmla_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, _sh(stream)))
            check(lib().qmla_stream_synchronize(_sh(stream)))
        return out

    def upload(self, a: np.ndarray, stream=None):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().qmla_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, _sh(stream)))
        check(lib().qmla_stream_synchronize(_sh(stream)))

    def zero(self, stream=None):
        check(lib().qmla_memset_zero(self.ptr, self.nbytes, _sh(stream)))

    def free(self):
        if self.ptr:
            lib().qmla_buffer_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _sh(stream):
    if stream is None:
        return None
    return stream.handle if isinstance(stream, Stream) else stream


def _p(x):
    if x is None:
        return None
    return x.ptr if isinstance(x, DeviceBuffer) else x


# --------------------------------------------- attention_kernel.rs mirror

def fused_prefill_attn(q_nope, q_rope, k, k_rope, v, scale: float, causal: bool, *, dims: PrefillDims,
                       dtype: int, out, stream=None):
    """fused_prefill_attn (src/attention_kernel.rs:64-107) on device buffers."""
    check(lib().qmla_fused_prefill_attn(C.byref(dims), dtype, _p(q_nope), _p(q_rope), _p(k), _p(k_rope),
                                        _p(v), float(scale), int(causal), _p(out), _sh(stream)))


def prefill_numpy(q_nope, q_rope, k, k_rope, v, scale: float, causal: bool, q_offset: int = 0,
                  dtype: int = F32) -> np.ndarray:
    """Host-array convenience wrapper: uploads, runs, downloads.
    dtype F32: float32 arrays; BF16: uint16 bf16 bit patterns."""
    b, h, sq, dn = q_nope.shape
    dr = q_rope.shape[-1] if q_rope is not None else 0
    sk, dv = k.shape[2], v.shape[-1]
    krh = k_rope.shape[1] if k_rope is not None else 1
    dims = PrefillDims(b, h, sq, sk, dn, dr, dv, krh, q_offset)
    npdt = _DT[dtype]
    bufs = [DeviceBuffer.from_numpy(np.ascontiguousarray(x, npdt)) if x is not None else None
            for x in (q_nope, q_rope, k, k_rope, v)]
    out = DeviceBuffer(b * h * sq * dv * np.dtype(npdt).itemsize)
    fused_prefill_attn(*bufs, scale, causal, dims=dims, dtype=dtype, out=out)
    check(lib().qmla_stream_synchronize(None))
    return out.to_numpy(npdt, (b, h, sq, dv))


def reference_eager_attn_numpy(q, k, v, scale: float, causal: bool, dtype: int = F32) -> np.ndarray:
    """reference_eager_attn (src/attention_kernel.rs:110-134) on host arrays."""
    b, h, s, d = q.shape
    dv = v.shape[-1]
    npdt = _DT[dtype]
    bq, bk, bv = (DeviceBuffer.from_numpy(np.ascontiguousarray(x, npdt)) for x in (q, k, v))
    out = DeviceBuffer(b * h * s * dv * np.dtype(npdt).itemsize)
    check(lib().qmla_reference_eager_attn(b, h, s, d, dv, dtype, bq.ptr, bk.ptr, bv.ptr, float(scale),
                                          int(causal), out.ptr, None))
    check(lib().qmla_stream_synchronize(None))
    return out.to_numpy(npdt, (b, h, s, dv))


# ------------------------------------------------------ KVCache mirror

class KVCache:
    """Latent KV cache (replaces KVCache, src/model.rs:86-105)."""

    def __init__(self, capacity, kv_lora_rank: int, rope_dim: int, dtype: int = BF16, _handle=None,
                 grow: bool = False, page_rows: int = 0, max_len: int = 0, pool_rows: int = 0):
        cap = np.ascontiguousarray(capacity, np.int32)
        self.num_seqs = int(cap.size)
        self.r, self.dr, self.dtype = kv_lora_rank, rope_dim, dtype
        if _handle is None:
            h = C.c_void_p()
            check(lib().qmla_cache_create_paged(self.num_seqs, cap.ctypes.data_as(C.POINTER(C.c_int32)),
                                                max_len, pool_rows, page_rows, kv_lora_rank, rope_dim,
                                                dtype, C.byref(h)))
            _handle = h.value
        self.handle = _handle
        if grow:
            self.set_growth(True)

    def reserve(self, min_capacity, stream=None):
        """Grow capacities to at least min_capacity (Tensor::cat never runs out of room)."""
        a = np.ascontiguousarray(min_capacity, np.int32)
        check(lib().qmla_cache_reserve(self.handle, a.ctypes.data_as(C.POINTER(C.c_int32)), _sh(stream)))

    def set_growth(self, enable: bool):
        check(lib().qmla_cache_set_growth(self.handle, 1 if enable else 0))

    def capacity(self) -> np.ndarray:
        out = np.empty(self.num_seqs, np.int32)
        check(lib().qmla_cache_capacity(self.handle, out.ctypes.data_as(C.POINTER(C.c_int32))))
        return out

    def append(self, rows, n_seqs: int, n_new: int, rows_dtype: int = F32, stream=None):
        check(lib().qmla_cache_append(self.handle, _p(rows), rows_dtype, n_seqs, n_new, _sh(stream)))

    def append_seq(self, seq: int, rows, n_new: int, rows_dtype: int = F32, stream=None):
        check(lib().qmla_cache_append_seq(self.handle, seq, _p(rows), rows_dtype, n_new, _sh(stream)))

    def set_lengths(self, lengths, stream=None):
        a = np.ascontiguousarray(lengths, np.int32)
        check(lib().qmla_cache_set_lengths(self.handle, a.ctypes.data_as(C.POINTER(C.c_int32)), _sh(stream)))

    def lengths(self) -> np.ndarray:
        out = np.empty(self.num_seqs, np.int32)
        check(lib().qmla_cache_lengths(self.handle, out.ctypes.data_as(C.POINTER(C.c_int32))))
        return out

    def describe(self) -> CacheDesc:
        d = CacheDesc()
        check(lib().qmla_cache_describe(self.handle, C.byref(d)))
        return d

    def clone(self, stream=None) -> "KVCache":
        h = C.c_void_p()
        check(lib().qmla_cache_clone(self.handle, C.byref(h), _sh(stream)))
        c = KVCache.__new__(KVCache)
        c.num_seqs, c.r, c.dr, c.dtype, c.handle = self.num_seqs, self.r, self.dr, self.dtype, h.value
        return c

    def _contiguous_desc(self) -> CacheDesc:
        d = self.describe()
        if not d.contiguous:
            raise QmlaError(2, "the cache's pages are no longer laid out in order; "
                                            "read sequences with read_seq")
        return d

    def read_rows(self) -> np.ndarray:
        """Whole creation-time chunk as numpy ([total_rows, r + dr], f32 or
        uint16); sequence i starts at row offsets()[i]."""
        d = self._contiguous_desc()
        npdt = _DT[d.dtype]
        out = np.empty((d.total_rows, d.row_elems), npdt)
        if out.nbytes:
            check(lib().qmla_memcpy_d2h(out.ctypes.data, d.rows, out.nbytes, None))
            check(lib().qmla_stream_synchronize(None))
        return out

    def write_pool(self, rows: np.ndarray):
        """Overwrite the creation-time chunk from a host array in the cache
        dtype: either the chunk itself ([total_rows, r + dr]) or the
        sequences' capacities back to back ([sum(capacity), r + dr],
        sequence i's rows first), which is spread to each sequence's offset."""
        d = self._contiguous_desc()
        a = np.ascontiguousarray(rows, _DT[d.dtype]).reshape(-1, d.row_elems)
        if a.shape[0] != d.total_rows:
            caps = self.capacity().astype(np.int64)
            assert a.shape[0] == caps.sum(), (a.shape, d.total_rows, caps.sum())
            pool = np.zeros((d.total_rows, d.row_elems), a.dtype)
            offs, src = self.offsets(), 0
            for i, c in enumerate(caps):
                pool[offs[i]:offs[i] + c] = a[src:src + c]
                src += c
            a = pool
        check(lib().qmla_memcpy_h2d(d.rows, a.ctypes.data, a.nbytes, None))
        check(lib().qmla_stream_synchronize(None))

    def read_seq(self, seq: int, n: int = None, t0: int = 0) -> np.ndarray:
        """Rows [t0, t0 + n) of one sequence (default: its live rows) as numpy,
        gathered through the block table ([n, r + dr], f32 or uint16)."""
        if n is None:
            n = int(self.lengths()[seq]) - t0
        out = np.empty((n, self.r + self.dr), _DT[self.dtype])
        if n:
            buf = DeviceBuffer(out.nbytes)
            check(lib().qmla_cache_gather(self.handle, seq, t0, n, _p(buf), None))
            check(lib().qmla_stream_synchronize(None))
            check(lib().qmla_memcpy_d2h(out.ctypes.data, _p(buf), out.nbytes, None))
        return out

    def trim(self, seq0: int = 0, n_seqs: int = None, stream=None):
        """Return pages beyond each listed sequence's length to the free list."""
        n_seqs = self.num_seqs - seq0 if n_seqs is None else n_seqs
        check(lib().qmla_cache_trim(self.handle, seq0, n_seqs, _sh(stream)))

    def reserve_pool(self, free_rows: int):
        """Top the free list up to at least free_rows rows (allocates now)."""
        check(lib().qmla_cache_reserve_pool(self.handle, free_rows))

    def pool_info(self):
        """(pool rows, free rows)."""
        a, b = C.c_int64(), C.c_int64()
        check(lib().qmla_cache_pool_info(self.handle, C.byref(a), C.byref(b)))
        return a.value, b.value

    def page_table(self) -> np.ndarray:
        """Host copy of the device block table [num_seqs, table_width] (uint64)."""
        d = self.describe()
        out = np.empty((self.num_seqs, d.table_width), np.uint64)
        check(lib().qmla_memcpy_d2h(out.ctypes.data, d.pages, out.nbytes, None))
        check(lib().qmla_stream_synchronize(None))
        return out

    def offsets(self) -> np.ndarray:
        d = self._contiguous_desc()
        out = np.empty(self.num_seqs, np.int64)
        check(lib().qmla_memcpy_d2h(out.ctypes.data, d.offsets, out.nbytes, None))
        check(lib().qmla_stream_synchronize(None))
        return out

    def close(self):
        if self.handle:
            lib().qmla_cache_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------ absorbed decode

def decode_workspace_bytes(cache: KVCache, batch: int, rows: int, splits: int = 0) -> int:
    dd = DecodeDims(batch, rows, cache.r, cache.dr)
    n = C.c_size_t()
    check(lib().qmla_decode_workspace_bytes_splits(C.byref(dd), cache.handle, splits, C.byref(n)))
    return n.value


def decode_absorbed(cache: KVCache, batch: int, rows: int, q_lat, q_rope, scale: float, out, lse=None,
                    q_dtype: int = F32, workspace=None, workspace_bytes: int = 0, splits: int = 0,
                    stream=None):
    dd = DecodeDims(batch, rows, cache.r, cache.dr)
    check(lib().qmla_decode_absorbed_splits(C.byref(dd), cache.handle, q_dtype, _p(q_lat), _p(q_rope),
                                            float(scale), _p(out), _p(lse), splits, _p(workspace),
                                            workspace_bytes, _sh(stream)))


def decode_numpy(cache: KVCache, q_lat: np.ndarray, q_rope: np.ndarray, scale: float, splits: int = 0,
                 q_dtype: int = F32):
    """q_lat [batch, rows, r], q_rope [batch, rows, dr] host arrays -> (out, lse)."""
    batch, rows, r = q_lat.shape
    npdt = _DT[q_dtype]
    bq = DeviceBuffer.from_numpy(np.ascontiguousarray(q_lat, npdt))
    br = DeviceBuffer.from_numpy(np.ascontiguousarray(q_rope, npdt))
    out = DeviceBuffer(batch * rows * r * 4)
    lse = DeviceBuffer(batch * rows * 4)
    wsb = decode_workspace_bytes(cache, batch, rows, splits)
    ws = DeviceBuffer(wsb)
    decode_absorbed(cache, batch, rows, bq, br, scale, out, lse, q_dtype, ws, wsb, splits)
    check(lib().qmla_stream_synchronize(None))
    return out.to_numpy(np.float32, (batch, rows, r)), lse.to_numpy(np.float32, (batch, rows))


# ------------------------------------------------------ MlaAttention mirror

class MlaLayer:
    """MlaAttention (src/model.rs:107-307) with device-resident f32 weights."""

    def __init__(self, w):
        """w: an object with hidden, heads, dn, dr, dv, r and the weight
        arrays wq, bq, wkva, bkva, ln_w, ln_b, wkvb, bkvb, wo, bo (f32)."""
        cfg = LayerConfig(w.hidden, w.heads, w.dn, w.dr, w.dv, w.r, 0.0, 0.0, 0.0)
        check(lib().qmla_layer_default_scales(C.byref(cfg)))
        if getattr(w, "softmax_scale", None) is not None:
            cfg.softmax_scale = float(w.softmax_scale)
        self.cfg = cfg
        keep = [np.ascontiguousarray(getattr(w, n), np.float32) if getattr(w, n) is not None else None
                for n in ("wq", "bq", "wkva", "bkva", "ln_w", "ln_b", "wkvb", "bkvb", "wo", "bo")]
        h = C.c_void_p()
        check(lib().qmla_layer_create(C.byref(cfg), *[a.ctypes.data if a is not None else None for a in keep],
                                      C.byref(h)))
        self.handle = h.value
        self.hidden = w.hidden

    def set_projection_dtype(self, dtype: int) -> None:
        """F32 (default): f32-exact projections; BF16: bf16 operands with f32
        accumulation in the hand-written projection kernels."""
        check(lib().qmla_layer_set_projection_dtype(self.handle, dtype))

    def workspace_bytes(self, cache: KVCache, batch: int, seq: int) -> int:
        """Scratch that serves either forward call for (batch, seq) tokens."""
        n = C.c_size_t()
        check(lib().qmla_layer_workspace_bytes(self.handle, cache.handle, batch, seq, C.byref(n)))
        return n.value

    def prefill_workspace_bytes(self, cache: KVCache, batch: int, seq: int) -> int:
        """Scratch that forward_prefill alone needs for (batch, seq) tokens."""
        n = C.c_size_t()
        check(lib().qmla_layer_prefill_workspace_bytes(self.handle, cache.handle, batch, seq, C.byref(n)))
        return n.value

    def forward_with_cache(self, xs: np.ndarray, cache: KVCache, stream=None) -> np.ndarray:
        b, s, _ = xs.shape
        bx = DeviceBuffer.from_numpy(np.ascontiguousarray(xs, np.float32))
        out = DeviceBuffer(b * s * self.hidden * 4)
        wsb = self.workspace_bytes(cache, b, s)
        ws = DeviceBuffer(wsb)
        check(lib().qmla_layer_forward_with_cache(self.handle, bx.ptr, b, s, cache.handle, out.ptr, ws.ptr,
                                                  wsb, _sh(stream)))
        check(lib().qmla_stream_synchronize(_sh(stream)))
        return out.to_numpy(np.float32, (b, s, self.hidden))

    def forward_prefill(self, xs: np.ndarray, cache: KVCache, stream=None) -> np.ndarray:
        b, s, _ = xs.shape
        bx = DeviceBuffer.from_numpy(np.ascontiguousarray(xs, np.float32))
        out = DeviceBuffer(b * s * self.hidden * 4)
        wsb = self.prefill_workspace_bytes(cache, b, s)
        ws = DeviceBuffer(wsb)
        check(lib().qmla_layer_forward_prefill(self.handle, bx.ptr, b, s, cache.handle, out.ptr, ws.ptr,
                                               wsb, _sh(stream)))
        check(lib().qmla_stream_synchronize(_sh(stream)))
        return out.to_numpy(np.float32, (b, s, self.hidden))

    def materialise(self, cache: KVCache, seq0: int = 0, n_seqs: int | None = None):
        """The reference KVCache's public tensors (src/model.rs:88-92) for
        sequences seq0 .. seq0 + n_seqs - 1 of one length T, rebuilt through
        kv_b_proj: (k [n, H, T, dn], v [n, H, T, dv], k_rope [n, H, T, dr])."""
        n = cache.num_seqs - seq0 if n_seqs is None else n_seqs
        nb = C.c_size_t()
        check(lib().qmla_cache_materialise_workspace_bytes(self.handle, cache.handle, seq0, n, C.byref(nb)))
        T = int(cache.lengths()[seq0])
        c = self.cfg
        H, dn, dv, dr = c.heads, c.qk_nope, c.v_dim, c.qk_rope
        k = DeviceBuffer(n * H * T * dn * 4)
        v = DeviceBuffer(n * H * T * dv * 4)
        kr = DeviceBuffer(n * H * T * dr * 4)
        ws = DeviceBuffer(nb.value) if nb.value else None
        check(lib().qmla_cache_materialise(self.handle, cache.handle, seq0, n, k.ptr, v.ptr, kr.ptr, _p(ws),
                                           nb.value, None))
        check(lib().qmla_stream_synchronize(None))
        return (k.to_numpy(np.float32, (n, H, T, dn)), v.to_numpy(np.float32, (n, H, T, dv)),
                kr.to_numpy(np.float32, (n, H, T, dr)))

    def close(self):
        if self.handle:
            lib().qmla_layer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# --------------------------------------------- tensor.rs / moe.rs mirror

def packed_workspace_bytes(out_features: int, in_features: int, batch: int) -> int:
    n = C.c_size_t()
    check(lib().qmla_packed_forward_workspace_bytes(out_features, in_features, batch, C.byref(n)))
    return n.value


class PackedQMoETensor:
    """PackedQMoETensor (src/tensor.rs:16-122) with its bytes and scales in
    HBM: shape (out_features, in_features), in_features / 4 bytes a row."""

    def __init__(self, packed, shape, scales):
        out_f, in_f = shape
        self.shape = (int(out_f), int(in_f))
        p = np.ascontiguousarray(packed, np.uint8).reshape(-1)
        sc = np.ascontiguousarray(scales, np.float32).reshape(-1)
        if p.size < out_f * (in_f // 4) or sc.size < out_f:
            raise QmlaError(2, "packed bytes or scales smaller than the shape")
        self.data = DeviceBuffer.from_numpy(p)
        self.scales = DeviceBuffer.from_numpy(sc)

    @staticmethod
    def from_bytes(packed, shape, scales) -> "PackedQMoETensor":
        return PackedQMoETensor(packed, shape, scales)

    def forward(self, x, batch: int, out, workspace=None, workspace_bytes: int = 0, stream=None):
        """Device form: x [batch, in] f32 -> out [batch, out] f32 (buffers)."""
        check(lib().qmla_packed_forward(self.data.ptr, self.scales.ptr, self.shape[0], self.shape[1], _p(x),
                                        batch, _p(out), _p(workspace), workspace_bytes, _sh(stream)))

    def forward_simd(self, x: np.ndarray) -> np.ndarray:
        """forward_simd (src/tensor.rs:64-95): x [..., in] -> [..., out]."""
        out_f, in_f = self.shape
        x = np.ascontiguousarray(x, np.float32)
        if in_f == 0 or x.size % in_f:
            raise QmlaError(2, f"input size {x.size} is not a multiple of in_features {in_f}")
        batch = x.size // in_f
        bx = DeviceBuffer.from_numpy(x)
        out = DeviceBuffer(batch * out_f * 4)
        n = packed_workspace_bytes(out_f, in_f, batch)
        ws = DeviceBuffer(n) if n else None
        self.forward(bx, batch, out, ws, n)
        check(lib().qmla_stream_synchronize(None))
        return out.to_numpy(np.float32, x.shape[:-1] + (out_f,))


class QMoELayer:
    """QMoELayer (src/moe.rs:23-131).  experts: a list of (gate, up, down)
    triples of (packed bytes, scales) host arrays, stacked into one HBM array
    per kind."""

    def __init__(self, config: MoEConfig, gate_weight: np.ndarray, experts):
        self.config = config
        E, H, I = config.num_experts, config.hidden_dim, config.intermediate_dim
        if len(experts) != E:
            raise QmlaError(2, f"{len(experts)} experts for num_experts {E}")
        kinds = list(zip(*experts)) if E else [(), (), ()]
        shapes = [(I, H), (I, H), (H, I)]
        self.bufs = []
        for kind, (o, i) in zip(kinds, shapes):
            pk = np.zeros((max(E, 1), o, i // 4), np.uint8)
            sc = np.zeros((max(E, 1), o), np.float32)
            for e, (p, s_) in enumerate(kind):
                pk[e] = np.asarray(p, np.uint8).reshape(o, i // 4)
                sc[e] = np.asarray(s_, np.float32).reshape(o)
            self.bufs += [DeviceBuffer.from_numpy(pk), DeviceBuffer.from_numpy(sc)]
        self.gate_weight = DeviceBuffer.from_numpy(np.ascontiguousarray(gate_weight, np.float32).reshape(-1)
                                                   if E else np.zeros(1, np.float32))

    def workspace_bytes(self, seq_len: int) -> int:
        n = C.c_size_t()
        check(lib().qmla_moe_workspace_bytes(C.byref(self.config), seq_len, C.byref(n)))
        return n.value

    def forward_device(self, xs, seq_len: int, out, workspace, workspace_bytes: int, top_experts=None,
                       top_weights=None, stream=None):
        gp, gs, up, us, dp, ds = (b.ptr for b in self.bufs)
        check(lib().qmla_moe_forward(C.byref(self.config), _p(xs), seq_len, self.gate_weight.ptr, gp, gs, up, us,
                                     dp, ds, _p(out), _p(top_experts), _p(top_weights), _p(workspace),
                                     workspace_bytes, _sh(stream)))

    def forward(self, xs: np.ndarray, return_routing: bool = False):
        """forward (src/moe.rs:40-130): xs [seq_len, hidden] -> [seq_len, hidden]."""
        xs = np.ascontiguousarray(xs, np.float32)
        T, H, k = xs.shape[0], self.config.hidden_dim, self.config.top_k
        bx = DeviceBuffer.from_numpy(xs)
        out = DeviceBuffer(T * H * 4)
        n = self.workspace_bytes(T)
        ws = DeviceBuffer(n)
        ti, tw = DeviceBuffer(T * max(k, 1) * 4), DeviceBuffer(T * max(k, 1) * 4)
        self.forward_device(bx, T, out, ws, n, ti, tw)
        check(lib().qmla_stream_synchronize(None))
        y = out.to_numpy(np.float32, (T, H))
        if return_routing:
            return y, ti.to_numpy(np.int32, (T, k)), tw.to_numpy(np.float32, (T, k))
        return y


# ------------------------------------------------------ HIP events (timing)

_hip = None


def hip_runtime():
    """libamdhip64 for event timing on a chosen stream."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        _hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        _hip.hipEventSynchronize.argtypes = [C.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        _hip.hipEventDestroy.argtypes = [C.c_void_p]
    return _hip


class Event:
    def __init__(self):
        h = C.c_void_p()
        if hip_runtime().hipEventCreate(C.byref(h)) != 0:
            raise RuntimeError("hipEventCreate failed")
        self.h = h.value

    def record(self, stream=None):
        if hip_runtime().hipEventRecord(self.h, _sh(stream)) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_ms(self, later: "Event") -> float:
        hip_runtime().hipEventSynchronize(later.h)
        t = C.c_float()
        if hip_runtime().hipEventElapsedTime(C.byref(t), self.h, later.h) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return t.value
