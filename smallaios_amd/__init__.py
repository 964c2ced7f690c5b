"""smallaios_amd -- MI355X (gfx950) compressed-KV GroupQueryAttention path.

Python binding (ctypes) of ``libsai_hip.so``, the C ABI declared in
``include/sai_hip.h``. Device buffers are passed as raw pointers; torch
tensors on ``cuda`` are accepted for convenience (torch is only used for
device memory and streams). Importing this package never falls back to a CPU
implementation: if the library is missing every call raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsai_hip.so")

SAI_OK = 0
STATUS_NAMES = {
    -1: "InvalidAttribute", -2: "ShapeMismatch", -3: "Unsupported", -4: "HipError",
    -5: "AllocFailed", -6: "PositionOverflow", -7: "NullArgument",
}
DTYPE_F32 = 1
DTYPE_F16 = 10
DTYPE_BF16 = 16
KV_INT8 = 1
KV_INT4 = 2
PAGE_TOKENS = 16

_lib = None


class SaiError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = STATUS_NAMES.get(status, f"status {status}")
        super().__init__(f"{self.kind}: {message}")


class _Desc(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int32), ("num_kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("num_pages", C.c_int32), ("max_batch", C.c_int32), ("max_pages_per_seq", C.c_int32),
        ("quant", C.c_int32),
    ]


class _TqDesc(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int32), ("num_kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("bits", C.c_int32), ("qjl", C.c_int32), ("max_batch", C.c_int32),
        ("max_rows", C.c_int32), ("seed", C.c_uint64), ("lowrank_k", C.c_int32),
    ]


def lib() -> C.CDLL:
    """Load libsai_hip.so (built in-tree by smallaios_amd/build.py)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python smallaios_amd/build.py` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        try:
            # torch bundles its own HIP runtime under the same soname
            # (libamdhip64.so.7); loading it first makes the process use one
            # runtime for torch tensors and this library alike
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        _declare(L)
        _lib = L
    return _lib


EXPORTS = [
    "sai_init", "sai_destroy", "sai_last_error", "sai_default_scale", "sai_device_supported",
    "sai_kvcache_create", "sai_kvcache_destroy", "sai_kvcache_set_page_table",
    "sai_kvcache_set_seq_lens", "sai_kvcache_advance", "sai_kvcache_reset",
    "sai_kvcache_lengths", "sai_kvcache_read", "sai_kvcache_pool", "sai_kv_append",
    "sai_kvcache_set_layer_window",
    "sai_gqa_decode", "sai_gqa_with_cache", "sai_gqa_with_cache_noalloc", "sai_gqa_prefill",
    "sai_set_decode_split",
    "sai_set_decode_waves", "sai_set_decode_merge", "sai_set_decode_reproducible",
    "sai_last_decode_shape",
    "sai_last_decode_launches",
    "sai_set_decode_timing", "sai_decode_kernel_times", "sai_rotary_embedding",
    "sai_rope_tables", "sai_copy_rows", "sai_tqcache_create", "sai_tqcache_destroy",
    "sai_tqcache_write", "sai_tqcache_advance", "sai_tqcache_reset", "sai_tqcache_set_lengths",
    "sai_tqcache_lengths", "sai_tqcache_read", "sai_tqcache_read_raw", "sai_tqcache_attend",
    "sai_tqcache_memory_bytes", "sai_tqcache_attention_logits", "sai_tqcache_weighted_value_sum",
    "sai_tqcache_write_attend", "sai_set_tq_split", "sai_tqcache_read_lowrank",
]
ROPE_BHSD = 0
ROPE_BSHD = 1


def _declare(L: C.CDLL) -> None:
    p, i32, f = C.c_void_p, C.c_int32, C.c_float
    pp = C.POINTER(C.c_void_p)
    sig = {
        "sai_init": (i32, [C.c_int, pp]),
        "sai_destroy": (None, [p]),
        "sai_last_error": (C.c_char_p, [p]),
        "sai_default_scale": (f, [i32]),
        "sai_device_supported": (i32, [C.c_int]),
        "sai_kvcache_create": (i32, [p, C.POINTER(_Desc), pp]),
        "sai_kvcache_destroy": (None, [p]),
        "sai_kvcache_set_page_table": (i32, [p, p, p, i32]),
        "sai_kvcache_set_seq_lens": (i32, [p, p, p, i32]),
        "sai_kvcache_advance": (i32, [p, p, p]),
        "sai_kvcache_reset": (i32, [p, p]),
        "sai_kvcache_lengths": (i32, [p, p, p, p]),
        "sai_kvcache_read": (i32, [p, p, i32, i32, i32, i32, i32, p, p, p, p]),
        "sai_kvcache_pool": (i32, [p, i32, pp, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
        "sai_kv_append": (i32, [p, p, i32, p, p, i32, i32, i32, p, p, i32, i32, i32, p]),
        "sai_gqa_decode": (i32, [p, p, i32, p, i32, i32, i32, p, p, i32, i32, i32, i32, f, i32,
                                 p, i32, p]),
        "sai_gqa_with_cache": (i32, [p, p, i32, p, i32, p, p, i32, i32, i32, p, p, i32, i32,
                                     i32, i32, f, i32, p, i32, p]),
        "sai_gqa_with_cache_noalloc": (i32, [p, p, i32, p, i32, p, p, i32, i32, i32, p, p, i32,
                                             i32, i32, i32, f, i32, p, i32, p]),
        "sai_gqa_prefill": (i32, [p, p, i32, p, i32, i32, i32, i32, p, p, i32, i32, i32, i32,
                                  f, i32, p, i32, p]),
        "sai_kvcache_set_layer_window": (i32, [p, p, i32, i32]),
        "sai_set_decode_split": (i32, [p, i32]),
        "sai_set_tq_split": (i32, [p, i32]),
        "sai_set_decode_waves": (i32, [p, i32]),
        "sai_set_decode_merge": (i32, [p, i32]),
        "sai_set_decode_reproducible": (i32, [p, i32]),
        "sai_last_decode_shape": (i32, [p, C.POINTER(i32), C.POINTER(i32)]),
        "sai_last_decode_launches": (i32, [p]),
        "sai_set_decode_timing": (i32, [p, i32]),
        "sai_decode_kernel_times": (i32, [p, C.POINTER(C.c_float), i32]),
        "sai_rotary_embedding": (i32, [p, p, p, i32, i32, i32, i32, i32, i32, p, C.c_int64,
                                       C.c_int64, p, p, i32, i32, i32, i32, i32, p]),
        "sai_rope_tables": (i32, [p, f, i32, i32, i32, p, p, p]),
        "sai_copy_rows": (i32, [p, p, i32, p, i32, i32, i32, i32, i32, i32, i32, i32, p]),
        "sai_tqcache_create": (i32, [p, C.POINTER(_TqDesc), pp]),
        "sai_tqcache_destroy": (None, [p]),
        "sai_tqcache_write": (i32, [p, p, i32, p, p, i32, i32, i32, p]),
        "sai_tqcache_advance": (i32, [p, p, p]),
        "sai_tqcache_reset": (i32, [p, p]),
        "sai_tqcache_set_lengths": (i32, [p, p, p, i32]),
        "sai_tqcache_lengths": (i32, [p, p, p, p]),
        "sai_tqcache_read": (i32, [p, p, i32, i32, i32, i32, i32, p, p]),
        "sai_tqcache_read_raw": (i32, [p, p, i32, i32, i32, i32, i32, p, p, p, p, p, p]),
        "sai_tqcache_read_lowrank": (i32, [p, p, i32, i32, i32, i32, i32, p, p]),
        "sai_tqcache_attend": (i32, [p, p, i32, p, i32, i32, i32, i32, f, p, p]),
        "sai_tqcache_memory_bytes": (i32, [p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
        "sai_tqcache_attention_logits": (i32, [p, p, i32, p, i32, i32, i32, p, i32, p]),
        "sai_tqcache_weighted_value_sum": (i32, [p, p, i32, p, i32, i32, i32, p, p]),
        "sai_tqcache_write_attend": (i32, [p, p, i32, p, i32, p, p, i32, i32, i32, i32, f, p, p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def default_scale(head_dim: int) -> float:
    return float(lib().sai_default_scale(head_dim))


def rope_tables(max_seq: int, head_dim: int, theta: float):
    """cos/sin caches [max_seq, head_dim/2] f32 (the op's cos_cache/sin_cache
    inputs): theta^(-2i/D) and cos/sin of pos * inv_freq in f64, rounded once."""
    half = head_dim // 2
    inv = theta ** (-(2.0 * np.arange(half, dtype=np.float64)) / head_dim)
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _dev_ptr(x):
    """Raw device pointer of a torch tensor / int / None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _dtype_code(x, default=DTYPE_F32):
    try:
        import torch
        if isinstance(x, torch.Tensor):
            return {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16,
                    torch.float16: DTYPE_F16}[x.dtype]
    except ImportError:  # pragma: no cover
        pass
    return default


def _stream(stream):
    if stream is None:
        try:
            import torch
            return torch.cuda.current_stream().cuda_stream
        except Exception:  # pragma: no cover
            return None
    return stream if isinstance(stream, int) else stream.cuda_stream


class Runtime:
    """sai_ctx: one per device."""

    def __init__(self, device: int = 0):
        self._L = lib()
        h = C.c_void_p()
        st = self._L.sai_init(device, C.byref(h))
        if st != SAI_OK:
            raise SaiError(st, f"sai_init({device})")
        self.handle = h
        self.device = device

    def close(self):
        if self.handle:
            self._L.sai_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def last_error(self) -> str:
        return self._L.sai_last_error(self.handle).decode()

    def check(self, st: int, what: str):
        if st != SAI_OK:
            raise SaiError(st, f"{what}: {self.last_error()}")

    def set_decode_split(self, tokens: int) -> int:
        return int(self._L.sai_set_decode_split(self.handle, tokens))

    def set_tq_split(self, rows: int) -> int:
        return int(self._L.sai_set_tq_split(self.handle, int(rows)))

    def set_decode_waves(self, waves: int) -> int:
        return int(self._L.sai_set_decode_waves(self.handle, waves))

    def set_decode_merge(self, mode) -> int:
        """0 / False: combine kernel, 1 / True: in-kernel merge, 2: automatic."""
        return int(self._L.sai_set_decode_merge(self.handle, int(mode)))

    def set_decode_reproducible(self, mode) -> int:
        """Tile order of the int8 decode and the TurboQuant attention: 1 / True
        fixed in both (bit-identical outputs across calls), 0 / False run-time
        hand-out in both, 2 (the default) fixed in the int8 decode only."""
        return int(self._L.sai_set_decode_reproducible(self.handle, int(mode)))

    def last_decode_shape(self):
        wg, sp = C.c_int32(), C.c_int32()
        self._L.sai_last_decode_shape(self.handle, C.byref(wg), C.byref(sp))
        return wg.value, sp.value

    def last_decode_launches(self) -> int:
        """Kernel launches of the last decode call: 1 (decode kernel) or 2
        (plus the combine kernel)."""
        return int(self._L.sai_last_decode_launches(self.handle))

    def set_decode_timing(self, slots: int) -> int:
        """HIP events around the decode kernel alone for the last `slots`
        decode calls (0 = off)."""
        return int(self._L.sai_set_decode_timing(self.handle, int(slots)))

    def decode_kernel_times(self, max_n: int):
        """Decode-kernel durations (us) of the most recent timed calls."""
        buf = (C.c_float * max_n)()
        n = self._L.sai_decode_kernel_times(self.handle, buf, max_n)
        if n < 0:
            self.check(n, "sai_decode_kernel_times")
        return [float(buf[i]) for i in range(n)]


    # ---- standalone RoPE --------------------------------------------------
    def rotary_embedding(self, x, y, batch, num_heads, seq, head_dim, cos, sin, *,
                         position_ids=None, start_position=0, layout=ROPE_BHSD,
                         rotary_dim=0, interleaved=False, stream=None, dtype=None,
                         table_dtype=None):
        """sai_rotary_embedding: rotate x (device, F32/BF16) into y (may be x).
        position_ids: host int array of seq or batch*seq entries, or None for
        start_position + s. cos/sin: device [rows, cols] (F32 or BF16)."""
        dt = dtype if dtype is not None else _dtype_code(x)
        tdt = table_dtype if table_dtype is not None else _dtype_code(cos)
        rows, cols = int(cos.shape[0]), int(cos.shape[1])
        ids = None
        n_pos = 0
        if position_ids is not None:
            ids = np.ascontiguousarray(position_ids, dtype=np.int64).ravel()
            n_pos = ids.size
        self.check(self._L.sai_rotary_embedding(
            self.handle, _dev_ptr(x), _dev_ptr(y), dt, batch, num_heads, seq, head_dim, layout,
            None if ids is None else ids.ctypes.data_as(C.c_void_p), n_pos, int(start_position),
            _dev_ptr(cos), _dev_ptr(sin), tdt, rows, cols, int(rotary_dim), int(interleaved),
            _stream(stream)), "rotary_embedding")

    def copy_rows(self, src, src_layout, dst, dst_layout, batch, heads, seq, head_dim, dst_seq,
                  dst_offset=0, dtype=None, stream=None):
        """sai_copy_rows: rows (b, h, s) of src to (b, h, dst_offset + s) of dst."""
        dt = dtype if dtype is not None else _dtype_code(src)
        self.check(self._L.sai_copy_rows(self.handle, _dev_ptr(src), int(src_layout),
                                         _dev_ptr(dst), int(dst_layout), dt, batch, heads, seq,
                                         head_dim, dst_seq, dst_offset, _stream(stream)),
                   "copy_rows")

    def rope_tables(self, max_pos, half, theta, cos_out, sin_out, dtype=DTYPE_BF16,
                    stream=None):
        """sai_rope_tables: the Gemma loader's [max_pos, half] tables on the device."""
        self.check(self._L.sai_rope_tables(self.handle, float(theta), int(max_pos), int(half),
                                           int(dtype), _dev_ptr(cos_out), _dev_ptr(sin_out),
                                           _stream(stream)), "rope_tables")


class KvCache:
    """sai_kvcache: paged int8/int4 KV cache (mirror of the reference's GpuKvCache)."""

    def __init__(self, rt: Runtime, num_layers, num_kv_heads, head_dim, num_pages, max_batch,
                 max_pages_per_seq, quant=KV_INT8):
        self.rt = rt
        self._L = rt._L
        self.desc = _Desc(num_layers, num_kv_heads, head_dim, num_pages, max_batch,
                          max_pages_per_seq, quant)
        h = C.c_void_p()
        rt.check(self._L.sai_kvcache_create(rt.handle, C.byref(self.desc), C.byref(h)),
                 "kvcache_create")
        self.handle = h
        self.num_layers, self.kv_heads, self.head_dim = num_layers, num_kv_heads, head_dim
        self.quant = quant
        self.max_pages_per_seq = max_pages_per_seq

    def close(self):
        if self.handle:
            self._L.sai_kvcache_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def set_page_table(self, table):
        t = np.ascontiguousarray(table, dtype=np.int32)
        assert t.ndim == 2 and t.shape[1] == self.max_pages_per_seq
        self.rt.check(self._L.sai_kvcache_set_page_table(
            self.rt.handle, self.handle, t.ctypes.data_as(C.c_void_p), t.shape[0]),
            "set_page_table")
        self.batch = t.shape[0]

    def set_seq_lens(self, lens):
        a = np.ascontiguousarray(lens, dtype=np.int32)
        self.rt.check(self._L.sai_kvcache_set_seq_lens(
            self.rt.handle, self.handle, a.ctypes.data_as(C.c_void_p), a.size), "set_seq_lens")

    def advance(self, stream=None):
        self.rt.check(self._L.sai_kvcache_advance(self.rt.handle, self.handle, _stream(stream)),
                      "advance")

    def reset(self):
        self.rt.check(self._L.sai_kvcache_reset(self.rt.handle, self.handle), "reset")

    def set_layer_window(self, layer: int, window: int):
        """Sliding-window layer: its queries see their last `window` keys (0: global)."""
        self.rt.check(self._L.sai_kvcache_set_layer_window(self.rt.handle, self.handle, layer,
                                                           int(window)), "set_layer_window")

    def lengths(self):
        b = C.c_int32()
        pend = C.c_int32()
        self._L.sai_kvcache_lengths(self.handle, None, C.byref(pend), C.byref(b))
        out = np.zeros(max(b.value, 1), dtype=np.int32)
        self._L.sai_kvcache_lengths(self.handle, out.ctypes.data_as(C.c_void_p), None, None)
        return out[: b.value], pend.value

    def pool(self, layer: int):
        ptr, nbytes, bb = C.c_void_p(), C.c_size_t(), C.c_size_t()
        st = self._L.sai_kvcache_pool(self.handle, layer, C.byref(ptr), C.byref(nbytes),
                                      C.byref(bb))
        if st != SAI_OK:
            raise SaiError(st, "kvcache_pool")
        return ptr.value, nbytes.value, bb.value

    def read(self, layer, b, kv_head, t0, n):
        """Codes/params of tokens [t0, t0+n) in logical order (synchronous)."""
        D = self.head_dim
        if self.quant == KV_INT8:
            kc = np.zeros((n, D), np.int8)
            vc = np.zeros((n, D), np.int8)
            kp = np.zeros(n, np.float32)
            vp = np.zeros(n, np.float32)
        else:
            kc = np.zeros((n, D // 2), np.uint8)
            vc = np.zeros((n, D // 2), np.uint8)
            kp = np.zeros((n, D // 32, 2), np.uint16)
            vp = np.zeros((n, D // 32, 2), np.uint16)
        ptr = lambda a: a.ctypes.data_as(C.c_void_p)
        self.rt.check(self._L.sai_kvcache_read(self.rt.handle, self.handle, layer, b, kv_head, t0,
                                               n, ptr(kc), ptr(vc), ptr(kp), ptr(vp)),
                      "kvcache_read")
        return kc, vc, kp, vp

    # ---- kernels ----------------------------------------------------------
    def append(self, layer, k, v, batch, s_new, cos=None, sin=None, cache_rows=0,
               do_rotary=True, interleaved=False, stream=None, dtype=None):
        dt = dtype if dtype is not None else _dtype_code(k)
        self.rt.check(self._L.sai_kv_append(
            self.rt.handle, self.handle, layer, _dev_ptr(k), _dev_ptr(v), dt, batch, s_new,
            _dev_ptr(cos), _dev_ptr(sin), cache_rows, int(do_rotary), int(interleaved),
            _stream(stream)), "kv_append")

    def decode(self, layer, q, out, batch, num_heads, cos=None, sin=None, cache_rows=0,
               do_rotary=True, interleaved=False, scale=None, stream=None, dtype=None, window=0):
        """window: the node's local_window_size (> 0: keys [p - window, p])."""
        dt = dtype if dtype is not None else _dtype_code(q)
        self.rt.check(self._L.sai_gqa_decode(
            self.rt.handle, self.handle, layer, _dev_ptr(q), dt, batch, num_heads, _dev_ptr(cos),
            _dev_ptr(sin), cache_rows, int(do_rotary), int(interleaved), int(scale is not None),
            0.0 if scale is None else float(scale), int(window), _dev_ptr(out),
            _dtype_code(out), _stream(stream)), "gqa_decode")

    def decode_with_cache(self, layer, q, k_new, v_new, out, batch, num_heads, cos=None,
                          sin=None, cache_rows=0, do_rotary=True, interleaved=False, scale=None,
                          stream=None, q_dtype=None, kv_dtype=None, window=0):
        """Fused step: append the token (k_new/v_new [B,1,Hkv*D]) and attend."""
        qd = q_dtype if q_dtype is not None else _dtype_code(q)
        kd = kv_dtype if kv_dtype is not None else _dtype_code(k_new)
        self.rt.check(self._L.sai_gqa_with_cache(
            self.rt.handle, self.handle, layer, _dev_ptr(q), qd, _dev_ptr(k_new), _dev_ptr(v_new),
            kd, batch, num_heads, _dev_ptr(cos), _dev_ptr(sin), cache_rows, int(do_rotary),
            int(interleaved), int(scale is not None), 0.0 if scale is None else float(scale),
            int(window), _dev_ptr(out), _dtype_code(out), _stream(stream)), "gqa_with_cache")

    def decode_with_cache_noalloc(self, layer, q, k_new, v_new, out, batch, num_heads, cos=None,
                                  sin=None, cache_rows=0, do_rotary=True, interleaved=False,
                                  scale=None, stream=None, q_dtype=None, kv_dtype=None, window=0):
        """decode_with_cache over the library's fixed per-GPU scratch (no
        device allocation; calls overlapping on one GPU race)."""
        qd = q_dtype if q_dtype is not None else _dtype_code(q)
        kd = kv_dtype if kv_dtype is not None else _dtype_code(k_new)
        self.rt.check(self._L.sai_gqa_with_cache_noalloc(
            self.rt.handle, self.handle, layer, _dev_ptr(q), qd, _dev_ptr(k_new), _dev_ptr(v_new),
            kd, batch, num_heads, _dev_ptr(cos), _dev_ptr(sin), cache_rows, int(do_rotary),
            int(interleaved), int(scale is not None), 0.0 if scale is None else float(scale),
            int(window), _dev_ptr(out), _dtype_code(out), _stream(stream)),
            "gqa_with_cache_noalloc")

    def prefill(self, layer, q, out, batch, sq, num_heads, cos=None, sin=None, cache_rows=0,
                do_rotary=True, interleaved=False, scale=None, stream=None, dtype=None, window=0):
        dt = dtype if dtype is not None else _dtype_code(q)
        self.rt.check(self._L.sai_gqa_prefill(
            self.rt.handle, self.handle, layer, _dev_ptr(q), dt, batch, sq, num_heads,
            _dev_ptr(cos), _dev_ptr(sin), cache_rows, int(do_rotary), int(interleaved),
            int(scale is not None), 0.0 if scale is None else float(scale), int(window),
            _dev_ptr(out), _dtype_code(out), _stream(stream)), "gqa_prefill")


class TqCache:
    """sai_tqcache: the TurboQuant compressed KV cache (CompressedKVCache of
    kv_compression.rs) on the device."""

    def __init__(self, rt: Runtime, num_layers, num_kv_heads, head_dim, bits, qjl, max_batch,
                 max_rows, seed=0, lowrank_k=None):
        """lowrank_k: KVCacheConfig::kv_lowrank_k (None, or a rank; 0 counts as 1)."""
        self.rt = rt
        self._L = rt._L
        lr = 0 if lowrank_k is None else max(1, int(lowrank_k))
        self.desc = _TqDesc(num_layers, num_kv_heads, head_dim, bits, int(bool(qjl)), max_batch,
                            max_rows, seed & (2**64 - 1), lr)
        h = C.c_void_p()
        rt.check(self._L.sai_tqcache_create(rt.handle, C.byref(self.desc), C.byref(h)),
                 "tqcache_create")
        self.handle = h
        self.num_layers, self.kv_heads, self.head_dim = num_layers, num_kv_heads, head_dim
        self.bits, self.qjl, self.max_batch = bits, bool(qjl), max_batch

    def close(self):
        if self.handle:
            self._L.sai_tqcache_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def write(self, layer, k, v, batch, s_new, stream=None, dtype=None):
        """k, v: device [batch, s_new, kv_heads*head_dim] (f32 or bf16)."""
        dt = dtype if dtype is not None else _dtype_code(k)
        self.rt.check(self._L.sai_tqcache_write(self.rt.handle, self.handle, layer, _dev_ptr(k),
                                                _dev_ptr(v), dt, batch, s_new, _stream(stream)),
                      "tqcache_write")

    def advance(self, stream=None):
        self.rt.check(self._L.sai_tqcache_advance(self.rt.handle, self.handle, _stream(stream)),
                      "tqcache_advance")

    def reset(self):
        self.rt.check(self._L.sai_tqcache_reset(self.rt.handle, self.handle), "tqcache_reset")

    def set_lengths(self, lens):
        a = np.ascontiguousarray(lens, dtype=np.int32)
        self.rt.check(self._L.sai_tqcache_set_lengths(self.rt.handle, self.handle,
                                                      a.ctypes.data_as(C.c_void_p), a.size),
                      "tqcache_set_lengths")

    def lengths(self):
        out = np.zeros(self.max_batch, np.int32)
        pend, b = C.c_int32(), C.c_int32()
        self._L.sai_tqcache_lengths(self.handle, out.ctypes.data_as(C.c_void_p), C.byref(pend),
                                    C.byref(b))
        return out, pend.value, b.value

    def memory_bytes(self):
        """(the reference's memory_bytes of the committed rows, device bytes held)."""
        r, d = C.c_uint64(), C.c_uint64()
        st = self._L.sai_tqcache_memory_bytes(self.handle, C.byref(r), C.byref(d))
        if st != SAI_OK:
            raise SaiError(st, "tqcache_memory_bytes")
        return r.value, d.value

    def read(self, layer, b, kv_head, start, n):
        """Decoded rows (read_k, read_v), f32 [n, head_dim] each (synchronous)."""
        k = np.zeros((n, self.head_dim), np.float32)
        v = np.zeros((n, self.head_dim), np.float32)
        self.rt.check(self._L.sai_tqcache_read(self.rt.handle, self.handle, layer, b, kv_head,
                                               start, n, k.ctypes.data_as(C.c_void_p),
                                               v.ctypes.data_as(C.c_void_p)), "tqcache_read")
        return k, v

    def read_lowrank(self, layer, b, kv_head, start, n):
        """The low-rank K state (rank 1): (U_S [n] of rows start.., Vt [D])."""
        us = np.zeros(n, np.float32)
        vt = np.zeros(self.head_dim, np.float32)
        self.rt.check(self._L.sai_tqcache_read_lowrank(
            self.rt.handle, self.handle, layer, b, kv_head, start, n,
            us.ctypes.data_as(C.c_void_p), vt.ctypes.data_as(C.c_void_p)), "tqcache_read_lowrank")
        return us, vt

    def read_raw(self, layer, b, kv_head, start, n):
        """Stored rows: dict of k/v codes [n, D*bits/8] u8, params [n, 3] f32
        (scale, zero, C), signs [n, D/64] u64 (zeros without QJL)."""
        D = self.head_dim
        cb = D * self.bits // 8
        r = {"k_codes": np.zeros((n, cb), np.uint8), "v_codes": np.zeros((n, cb), np.uint8),
             "k_params": np.zeros((n, 3), np.float32), "v_params": np.zeros((n, 3), np.float32),
             "k_signs": np.zeros((n, D // 64), np.uint64),
             "v_signs": np.zeros((n, D // 64), np.uint64)}
        ptr = lambda key: r[key].ctypes.data_as(C.c_void_p)
        sk = ptr("k_signs") if self.qjl else None
        sv = ptr("v_signs") if self.qjl else None
        self.rt.check(self._L.sai_tqcache_read_raw(
            self.rt.handle, self.handle, layer, b, kv_head, start, n, ptr("k_codes"),
            ptr("v_codes"), ptr("k_params"), ptr("v_params"), sk, sv), "tqcache_read_raw")
        return r

    def write_attend(self, layer, q, k_new, v_new, out, batch, num_heads, scale=None,
                     stream=None, q_dtype=None, kv_dtype=None):
        """One decode step: store the new row (k_new/v_new [B, 1, Hkv*D]) and attend."""
        qd = q_dtype if q_dtype is not None else _dtype_code(q)
        kd = kv_dtype if kv_dtype is not None else _dtype_code(k_new)
        self.rt.check(self._L.sai_tqcache_write_attend(
            self.rt.handle, self.handle, layer, _dev_ptr(q), qd, _dev_ptr(k_new), _dev_ptr(v_new),
            kd, batch, num_heads, int(scale is not None), 0.0 if scale is None else float(scale),
            _dev_ptr(out), _stream(stream)), "tqcache_write_attend")

    def attention_logits(self, layer, q, logits, ld, batch, num_heads, stream=None, dtype=None):
        """logits: device f32 [batch * num_heads, ld] (unscaled inner-product estimates)."""
        dt = dtype if dtype is not None else _dtype_code(q)
        self.rt.check(self._L.sai_tqcache_attention_logits(
            self.rt.handle, self.handle, layer, _dev_ptr(q), dt, batch, num_heads,
            _dev_ptr(logits), int(ld), _stream(stream)), "tqcache_attention_logits")

    def weighted_value_sum(self, layer, weights, ld, out, batch, num_heads, stream=None):
        """weights: device f32 [batch * num_heads, ld]; out: device f32
        [batch, 1, num_heads * head_dim]."""
        self.rt.check(self._L.sai_tqcache_weighted_value_sum(
            self.rt.handle, self.handle, layer, _dev_ptr(weights), int(ld), batch, num_heads,
            _dev_ptr(out), _stream(stream)), "tqcache_weighted_value_sum")

    def attend(self, layer, q, out, batch, num_heads, scale=None, stream=None, dtype=None):
        """q: device [batch, 1, num_heads*head_dim]; out: device f32, same shape."""
        dt = dtype if dtype is not None else _dtype_code(q)
        self.rt.check(self._L.sai_tqcache_attend(
            self.rt.handle, self.handle, layer, _dev_ptr(q), dt, batch, num_heads,
            int(scale is not None), 0.0 if scale is None else float(scale), _dev_ptr(out),
            _stream(stream)), "tqcache_attend")


def identity_page_table(batch: int, pages_per_seq: int):
    """Sequence b owns pages [b*pages_per_seq, (b+1)*pages_per_seq)."""
    return np.arange(batch * pages_per_seq, dtype=np.int32).reshape(batch, pages_per_seq)
