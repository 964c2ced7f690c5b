"""CPU oracle (test infrastructure only).

Thin numpy/ctypes wrapper over ``libsai_oracle.so``, the C restatement of the
reference's Rust CPU semantics for the GroupQueryAttention + quantised KV path
(see ``sai_oracle.c`` for the file:line each function follows).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker. The product
library ``smallaios_amd/libsai_hip.so`` never loads it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libsai_oracle.so")
_lib = None

INT8 = 1
INT4 = 2


def build() -> str:
    """Compile the oracle with its Makefile (gcc, plain IEEE f32)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_f = C.c_float
_i = C.c_int
_p = C.c_void_p
_sz = C.c_size_t


def _declare(L: C.CDLL) -> None:
    sig = {
        "sai_or_expf_approx": (_f, [_f]),
        "sai_or_sqrt_f32": (_f, [_f]),
        "sai_or_sqrt_approx": (_f, [_f]),
        "sai_or_round_half_even": (_f, [_f]),
        "sai_or_round_f32_kv": (_f, [_f]),
        "sai_or_sat_i32": (C.c_int32, [_f]),
        "sai_or_sat_u32": (C.c_uint32, [_f]),
        "sai_or_f32_to_bf16": (C.c_uint16, [_f]),
        "sai_or_bf16_to_f32": (_f, [C.c_uint16]),
        "sai_or_f32_to_f16": (C.c_uint16, [_f]),
        "sai_or_f16_to_f32": (_f, [C.c_uint16]),
        "sai_or_f32_to_f16_array": (None, [_p, _sz, _p]),
        "sai_or_round_half_even_array": (None, [_p, _sz, _p]),
        "sai_or_expf_approx_array": (None, [_p, _sz, _p]),
        "sai_or_default_scale": (_f, [_i]),
        "sai_or_pack_bits": (None, [_p, _sz, _i, _p]),
        "sai_or_unpack_bits": (None, [_p, _sz, _sz, _i, _p]),
        "sai_or_apply_rope": (_i, [_p, _i, _i, _i, _i, _p, _p, _i, _i, _p, _i, _i, _i]),
        "sai_or_sdpa": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _f, _i, _p]),
        "sai_or_gqa": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _p, _i, _p, _p, _i, _i, _i, _i,
                            _i, _f, _i, _i, _i, _p, _p, _p]),
        "sai_or_quant_int8_row": (None, [_p, _i, _p, _p]),
        "sai_or_dequant_int8_row": (None, [_p, _f, _i, _p]),
        "sai_or_quant_int4_row": (None, [_p, _i, _p, _p, _p]),
        "sai_or_dequant_int4_row": (None, [_p, _p, _p, _i, _p]),
        "sai_or_kv_append": (_i, [_p, _p, _i, _i, _i, _i, _p, _p, _p, _i, _i, _i, _i, _i, _p,
                                  _p, _p, _p, _p, _p]),
        "sai_or_kv_dequant": (_i, [_i, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
        "sai_or_gqa_cached": (_i, [_p, _i, _i, _i, _i, _i, _p, _i, _p, _p, _p, _p, _i, _i, _i,
                                   _i, _f, _p]),
        "sai_or_gqa_cached_window": (_i, [_p, _i, _i, _i, _i, _i, _p, _i, _p, _p, _p, _p, _i, _i,
                                          _i, _i, _f, _i, _i, _p]),
        "sai_or_sdpa_window": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _f, _i, _i, _p]),
        "sai_or_check_rhe_vs_rint": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "sai_or_ln_approx": (_f, [_f]),
        "sai_or_exp_approx": (_f, [_f]),
        "sai_or_floor_approx": (_f, [_f]),
        "sai_or_sin_approx": (_f, [_f]),
        "sai_or_cos_approx": (_f, [_f]),
        "sai_or_rope_tables_bf16": (None, [_i, _i, _f, _p, _p]),
        "sai_or_tq_signs": (None, [C.c_uint64, _i, _p]),
        "sai_or_tq_head_seed": (C.c_uint64, [C.c_uint64, _i, _i, _i]),
        "sai_or_wht_with_signs": (None, [_p, _p, _i]),
        "sai_or_inverse_wht_with_signs": (None, [_p, _p, _i]),
        "sai_or_tq_encode": (_i, [_p, _i, _i, _p, _p, _p, _p, _p, _p]),
        "sai_or_tq_decode": (None, [_p, _i, _i, _f, _f, _p, _p]),
        "sai_or_qjl_encode": (None, [_p, _p, _i, _p, _p]),
        "sai_or_qjl_correction": (_f, [_p, _f, _p, _f, _i]),
        "sai_or_tq_write_row": (_i, [_p, _i, _i, _p, _i, _p, _p, _p, _p, _p]),
        "sai_or_tq_attend": (_i, [_p, _i, _i, _i, _i, _p, _i, _p, _p, _p, _p, _p, _p, _p, _p,
                                  _f, _p]),
        "sai_or_tq_attention_logits": (_i, [_p, _i, _i, _i, _i, _p, _i, _p, _p, _p, _p, _p, _p]),
        "sai_or_tq_weighted_value_sum": (None, [_p, _i, _i, _i, _p, _i, _p, _p, _p, _p]),
        "sai_or_lr_decompose": (_i, [_p, _i, _i, _i, _p, _p]),
        "sai_or_lr_reconstruct": (None, [_p, _p, _i, _i, _i, _p]),
        "sai_or_lr_update": (None, [_p, _p, _p, _i, _p, _p, _p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleError(RuntimeError):
    """Mirrors the reference's OpError: code -1 InvalidAttribute, -2 ShapeMismatch."""

    def __init__(self, code: int, what: str):
        kind = {-1: "InvalidAttribute", -2: "ShapeMismatch"}.get(code, f"code {code}")
        super().__init__(f"{what}: {kind}")
        self.code = code
        self.kind = kind


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise OracleError(rc, what)


# ---------------------------------------------------------------- scalars ---
def expf_approx(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().sai_or_expf_approx_array(_ptr(x), x.size, _ptr(out))
    return out


def round_half_even(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().sai_or_round_half_even_array(_ptr(x), x.size, _ptr(out))
    return out


def f32_to_f16_bits(x):
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().sai_or_f32_to_f16_array(_ptr(x), x.size, _ptr(out))
    return out


def f32_to_bf16_bits(x):
    x = _f32(x).ravel()
    return np.array([lib().sai_or_f32_to_bf16(float(v)) for v in x], dtype=np.uint16)


def bf16_bits_to_f32(b):
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def default_scale(head_dim: int) -> float:
    return float(np.float32(lib().sai_or_default_scale(head_dim)))


def pack_bits(values, bits: int):
    v = np.ascontiguousarray(values, dtype=np.uint32)
    out = np.empty((v.size * bits + 7) // 8, dtype=np.uint8)
    lib().sai_or_pack_bits(_ptr(v), v.size, bits, _ptr(out))
    return out


def unpack_bits(data, count: int, bits: int):
    d = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(count, dtype=np.uint32)
    lib().sai_or_unpack_bits(_ptr(d), d.size, count, bits, _ptr(out))
    return out


# ------------------------------------------------------------ RoPE tables ---
def rope_tables_bf16(max_pos: int, half: int, theta: float):
    """The Gemma loader's precomputed tables (gemma.rs:458-472): (cos, sin)
    as bf16 bit patterns, uint16 [max_pos, half]."""
    c = np.empty((max_pos, half), np.uint16)
    s = np.empty((max_pos, half), np.uint16)
    lib().sai_or_rope_tables_bf16(max_pos, half, float(theta), _ptr(c), _ptr(s))
    return c, s


def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round to nearest even, NaN kept quiet (tensor.rs:312-329)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.ascontiguousarray(x, dtype=np.float32))
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


# ------------------------------------------------------------- TurboQuant ---
def tq_signs(seed: int, dim: int) -> np.ndarray:
    """PolarQuantizer::new's sign flips (xorshift64), int8 [dim] of +-1."""
    s = np.empty(dim, np.int8)
    lib().sai_or_tq_signs(C.c_uint64(seed & (2**64 - 1)), dim, _ptr(s))
    return s


def tq_head_seed(seed: int, layer: int, num_kv_heads: int, head: int) -> int:
    return int(lib().sai_or_tq_head_seed(C.c_uint64(seed & (2**64 - 1)), layer, num_kv_heads,
                                         head))


def wht(x, signs, inverse=False):
    y = _f32(x).copy()
    sg = np.ascontiguousarray(signs, np.int8)
    f = lib().sai_or_inverse_wht_with_signs if inverse else lib().sai_or_wht_with_signs
    f(_ptr(y), _ptr(sg), y.size)
    return y


def tq_encode(x, bits: int, signs):
    """PolarQuantizer::encode -> (packed u8, scale, zero, min, max)."""
    x = _f32(x)
    d = x.size
    packed = np.zeros((d * bits + 7) // 8, np.uint8)
    sc, z, mn, mx = (C.c_float() for _ in range(4))
    sg = np.ascontiguousarray(signs, np.int8)
    rc = lib().sai_or_tq_encode(_ptr(x), d, bits, _ptr(sg), _ptr(packed), C.byref(sc),
                                C.byref(z), C.byref(mn), C.byref(mx))
    _check(rc, "tq_encode")
    return packed, sc.value, z.value, mn.value, mx.value


def tq_decode(packed, dim: int, bits: int, scale: float, zero: float, signs):
    out = np.empty(dim, np.float32)
    p = np.ascontiguousarray(packed, np.uint8)
    sg = np.ascontiguousarray(signs, np.int8)
    lib().sai_or_tq_decode(_ptr(p), dim, bits, float(scale), float(zero), _ptr(sg), _ptr(out))
    return out


def qjl_encode(original, approx):
    o, a = _f32(original), _f32(approx)
    bits = np.zeros(max(1, (o.size + 63) // 64), np.uint64)
    c = C.c_float()
    lib().sai_or_qjl_encode(_ptr(o), _ptr(a), o.size, _ptr(bits), C.byref(c))
    return bits, c.value


def qjl_correction(a_bits, a_c, b_bits, b_c, dim: int) -> float:
    a = np.ascontiguousarray(a_bits, np.uint64)
    b = np.ascontiguousarray(b_bits, np.uint64)
    return float(lib().sai_or_qjl_correction(_ptr(a), float(a_c), _ptr(b), float(b_c), dim))


def tq_write_rows(x, bits: int, signs, qjl: bool):
    """CompressedKVCache::write_kv over rows x [n, D]: (codes [n, D*bits/8],
    scale [n], zero [n], sign words [n, D/64], c [n])."""
    x = _f32(x)
    n, d = x.shape
    cb, w = (d * bits + 7) // 8, (d + 63) // 64
    codes = np.zeros((n, cb), np.uint8)
    sc = np.zeros(n, np.float32)
    z = np.zeros(n, np.float32)
    sb = np.zeros((n, w), np.uint64)
    c = np.zeros(n, np.float32)
    sg = np.ascontiguousarray(signs, np.int8)
    for t in range(n):
        st, zt, ct = C.c_float(), C.c_float(), C.c_float()
        row = np.ascontiguousarray(x[t])
        rc = lib().sai_or_tq_write_row(_ptr(row), d, bits, _ptr(sg), int(qjl),
                                       codes[t].ctypes.data_as(C.c_void_p), C.byref(st),
                                       C.byref(zt), sb[t].ctypes.data_as(C.c_void_p),
                                       C.byref(ct))
        _check(rc, "tq_write_row")
        sc[t], z[t], c[t] = st.value, zt.value, ct.value
    return codes, sc, z, sb, c


def tq_attend(q, bits, qjl, signs, k, v, scale):
    """Decode attention of q [G, D] over encoded rows k/v = tq_write_rows
    outputs; returns [G, D]."""
    q = _f32(q)
    g, d = q.shape
    kc, ks, kz, ksb, kcm = k
    vc, vs, vz, _, _ = v
    out = np.zeros((g, d), np.float32)
    sg = np.ascontiguousarray(signs, np.int8)
    rc = lib().sai_or_tq_attend(_ptr(q), g, d, bits, int(qjl), _ptr(sg), kc.shape[0],
                                _ptr(np.ascontiguousarray(kc)), _ptr(ks), _ptr(kz),
                                _ptr(np.ascontiguousarray(ksb)), _ptr(kcm),
                                _ptr(np.ascontiguousarray(vc)), _ptr(vs), _ptr(vz),
                                float(scale), _ptr(out))
    _check(rc, "tq_attend")
    return out


def tq_attention_logits(q, bits, qjl, signs, k):
    """The design's attention_logits over encoded rows k (tq_write_rows
    output): [G, rows] unscaled estimates."""
    q = _f32(q)
    g, d = q.shape
    kc, ks, kz, ksb, kcm = k
    n = kc.shape[0]
    out = np.zeros((g, n), np.float32)
    sg = np.ascontiguousarray(signs, np.int8)
    rc = lib().sai_or_tq_attention_logits(_ptr(q), g, d, bits, int(qjl), _ptr(sg), n,
                                          _ptr(np.ascontiguousarray(kc)), _ptr(ks), _ptr(kz),
                                          _ptr(np.ascontiguousarray(ksb)), _ptr(kcm), _ptr(out))
    _check(rc, "tq_attention_logits")
    return out


def tq_weighted_value_sum(weights, bits, signs, v):
    """The design's weighted_value_sum: [G, D] = weights [G, rows] x decoded v."""
    w = _f32(weights)
    g, n = w.shape
    vc, vs, vz, _, _ = v
    d = len(signs)
    out = np.zeros((g, d), np.float32)
    sg = np.ascontiguousarray(signs, np.int8)
    lib().sai_or_tq_weighted_value_sum(_ptr(w), g, d, bits, _ptr(sg), n,
                                       _ptr(np.ascontiguousarray(vc)), _ptr(vs), _ptr(vz),
                                       _ptr(out))
    return out


class LowRankK:
    """LowRankK (kv_compression.rs:425-445) with LowRankKeyDecomposer's
    decompose / update / reconstruct (:470-577); u_s kept with room for
    `capacity` rows."""

    def __init__(self, k, rank: int, capacity: int | None = None):
        k = _f32(k)
        rows, cols = k.shape
        cap = max(rows, capacity or rows)
        r = max(1, rank)
        self.u_s = np.zeros(cap * r, np.float32)
        self.vt = np.zeros(r * cols, np.float32)
        self.rank = int(lib().sai_or_lr_decompose(_ptr(np.ascontiguousarray(k)), rows, cols, rank,
                                                  _ptr(self.u_s), _ptr(self.vt)))
        self.rows, self.cols, self.write_counter = rows, cols, 0

    def update(self, row):
        row = _f32(row)
        assert row.size == self.cols
        if (self.rows + 1) * self.rank > self.u_s.size:
            self.u_s = np.concatenate([self.u_s, np.zeros(self.u_s.size + self.rank, np.float32)])
        rows, rank, wc = C.c_int(self.rows), C.c_int(self.rank), C.c_int(self.write_counter)
        lib().sai_or_lr_update(_ptr(self.u_s), _ptr(self.vt), C.byref(rows), self.cols,
                               C.byref(rank), C.byref(wc), _ptr(row))
        self.rows, self.rank, self.write_counter = rows.value, rank.value, wc.value

    def factors(self):
        """(U_S [rows, rank], Vt [rank, cols])."""
        return (self.u_s[:self.rows * self.rank].reshape(self.rows, self.rank).copy(),
                self.vt[:self.rank * self.cols].reshape(self.rank, self.cols).copy())

    def reconstruct(self):
        out = np.zeros((self.rows, self.cols), np.float32)
        lib().sai_or_lr_reconstruct(_ptr(self.u_s), _ptr(self.vt), self.rows, self.cols,
                                    self.rank, _ptr(out))
        return out


def tq_lowrank_rows(k, rank: int) -> LowRankK:
    """CompressedKVCache::write_kv's low-rank K state (kv_compression.rs:840-852)
    after rows k [n, D] in order: the first row decomposed alone, the rest
    appended by update."""
    k = _f32(k)
    lr = LowRankK(k[:1], rank, capacity=k.shape[0])
    for t in range(1, k.shape[0]):
        lr.update(k[t])
    return lr


# ------------------------------------------------------------ RoPE / SDPA ---
def apply_rope(x, cos, sin, position_ids, interleaved=False, rotary_dim=None):
    """x: [B, H, Sq, D] f32 (returns a rotated copy)."""
    x = _f32(x).copy()
    b, h, sq, d = x.shape
    cos = _f32(cos)
    sin = _f32(sin)
    pos = np.ascontiguousarray(position_ids, dtype=np.int64)
    rc = lib().sai_or_apply_rope(_ptr(x), b, h, sq, d, _ptr(cos), _ptr(sin), cos.shape[0],
                                 cos.shape[1], _ptr(pos), pos.size, int(interleaved),
                                 d if rotary_dim is None else rotary_dim)
    _check(rc, "apply_rope")
    return x


def sdpa_window(q, k, v, num_kv_heads, past_sk, scale, layer_window=0, mask_window=0):
    """Causal SDPA with the reference's window rules; q [B,Hq,Sq,D], k/v [B,Hk,Sk,D]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, hq, sq, d = q.shape
    sk = k.shape[2]
    out = np.zeros_like(q)
    rc = lib().sai_or_sdpa_window(_ptr(q), _ptr(k), _ptr(v), b, hq, num_kv_heads, sq, sk, d,
                                  past_sk, float(scale), int(layer_window), int(mask_window),
                                  _ptr(out))
    _check(rc, "sdpa_window")
    return out


def sdpa(q, k, v, num_kv_heads, past_sk, scale, causal):
    """q [B,Hq,Sq,D], k/v [B,Hk,Sk,D] -> out [B,Hq,Sq,D]."""
    q = _f32(q)
    k = _f32(k)
    v = _f32(v)
    b, hq, sq, d = q.shape
    sk = k.shape[2] if k.size else 0
    out = np.empty_like(q)
    rc = lib().sai_or_sdpa(_ptr(q), _ptr(k), _ptr(v), b, hq, num_kv_heads, sq, sk, d, past_sk,
                           float(scale), int(causal), _ptr(out))
    _check(rc, "sdpa")
    return out


def gqa(query, key, value, num_heads, kv_num_heads, past_key=None, past_value=None,
        cos=None, sin=None, scale=None, local_window_size=-1, do_rotary=True,
        rotary_interleaved=False):
    """op_group_query_attention on f32 arrays. Returns (attn, present_k, present_v)."""
    q = _f32(query)
    k = _f32(key)
    v = _f32(value)
    b, sq, qh = q.shape
    kvh = k.shape[2]
    if v.shape != k.shape:
        raise OracleError(-2, "gqa")
    past_sk = 0 if past_key is None else past_key.shape[2]
    pk = None if past_key is None else _f32(past_key)
    pv = None if past_value is None else _f32(past_value)
    if pv is not None and pv.shape[2] != past_sk:
        raise OracleError(-2, "gqa")
    hd = qh // num_heads if num_heads > 0 else 1
    total = past_sk + sq
    attn = np.zeros((b, sq, qh), dtype=np.float32)
    kvn = max(kv_num_heads, 1)
    pres_k = np.zeros((b, kvn, total, hd), dtype=np.float32)
    pres_v = np.zeros((b, kvn, total, hd), dtype=np.float32)
    cosa = None if cos is None else _f32(cos)
    sina = None if sin is None else _f32(sin)
    rows = 0 if cosa is None else cosa.shape[0]
    cols = 0 if cosa is None else cosa.shape[1]
    rc = lib().sai_or_gqa(_ptr(q), _ptr(k), _ptr(v), b, sq, qh, kvh, _ptr(pk), _ptr(pv), past_sk,
                          _ptr(cosa), _ptr(sina), rows, cols, num_heads, kv_num_heads,
                          int(scale is not None), 0.0 if scale is None else float(scale),
                          local_window_size, int(do_rotary), int(rotary_interleaved),
                          _ptr(attn), _ptr(pres_k), _ptr(pres_v))
    _check(rc, "gqa")
    return attn, pres_k, pres_v


# ------------------------------------------------------------ quantisers ---
def quant_int8_row(x):
    x = _f32(x)
    codes = np.empty(x.size, dtype=np.int8)
    s = np.zeros(1, dtype=np.float32)
    lib().sai_or_quant_int8_row(_ptr(x), x.size, _ptr(codes), _ptr(s))
    return codes, np.float32(s[0])


def quant_int4_row(x):
    x = _f32(x)
    d = x.size
    packed = np.empty(d // 2, dtype=np.uint8)
    sc = np.empty(d // 32, dtype=np.uint16)
    z = np.empty(d // 32, dtype=np.uint16)
    lib().sai_or_quant_int4_row(_ptr(x), d, _ptr(packed), _ptr(sc), _ptr(z))
    return packed, sc, z


def dequant_int4_row(packed, sc, z, d):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    sc = np.ascontiguousarray(sc, dtype=np.uint16)
    z = np.ascontiguousarray(z, dtype=np.uint16)
    out = np.empty(d, dtype=np.float32)
    lib().sai_or_dequant_int4_row(_ptr(packed), _ptr(sc), _ptr(z), d, _ptr(out))
    return out


class LogicalCache:
    """Logical (un-paged) quantised KV cache in the oracle's layout.

    int8: codes [B, Hkv, T, D] int8, scales [B, Hkv, T] f32.
    int4: codes [B, Hkv, T, D/2] u8, sz [B, Hkv, T, D/32, 2] f16 bits (scale, zero).
    """

    def __init__(self, b, kv_heads, head_dim, t_cap, quant=INT8):
        self.b, self.kv_heads, self.head_dim, self.t_cap, self.quant = (
            b, kv_heads, head_dim, t_cap, quant)
        if quant == INT8:
            self.k_codes = np.zeros((b, kv_heads, t_cap, head_dim), dtype=np.int8)
            self.v_codes = np.zeros_like(self.k_codes)
            self.k_scale = np.zeros((b, kv_heads, t_cap), dtype=np.float32)
            self.v_scale = np.zeros_like(self.k_scale)
            self.k_sz = self.v_sz = None
        else:
            self.k_codes = np.zeros((b, kv_heads, t_cap, head_dim // 2), dtype=np.uint8)
            self.v_codes = np.zeros_like(self.k_codes)
            self.k_sz = np.zeros((b, kv_heads, t_cap, head_dim // 32, 2), dtype=np.uint16)
            self.v_sz = np.zeros_like(self.k_sz)
            self.k_scale = self.v_scale = None
        self.seq_len = np.zeros(b, dtype=np.int32)

    def append(self, k_new, v_new, cos=None, sin=None, do_rotary=True, interleaved=False):
        """k_new/v_new [B, S_new, Hkv*D] f32; appends at seq_len[b] and advances."""
        k = _f32(k_new)
        v = _f32(v_new)
        b, s_new, _ = k.shape
        start = np.ascontiguousarray(self.seq_len, dtype=np.int32)
        cosa = None if cos is None else _f32(cos)
        sina = None if sin is None else _f32(sin)
        rows = 0 if cosa is None else cosa.shape[0]
        rc = lib().sai_or_kv_append(_ptr(k), _ptr(v), b, s_new, self.kv_heads, self.head_dim,
                                    _ptr(start), _ptr(cosa), _ptr(sina), rows, int(do_rotary),
                                    int(interleaved), self.quant, self.t_cap, _ptr(self.k_codes),
                                    _ptr(self.v_codes), _ptr(self.k_scale), _ptr(self.v_scale),
                                    _ptr(self.k_sz), _ptr(self.v_sz))
        _check(rc, "kv_append")
        self.seq_len = self.seq_len + s_new

    def dequant(self):
        kd = np.zeros((self.b, self.kv_heads, self.t_cap, self.head_dim), dtype=np.float32)
        vd = np.zeros_like(kd)
        sl = np.ascontiguousarray(self.seq_len, dtype=np.int32)
        rc = lib().sai_or_kv_dequant(self.b, self.kv_heads, self.head_dim, self.quant, self.t_cap,
                                     _ptr(sl), _ptr(self.k_codes), _ptr(self.v_codes),
                                     _ptr(self.k_scale), _ptr(self.v_scale), _ptr(self.k_sz),
                                     _ptr(self.v_sz), _ptr(kd), _ptr(vd))
        _check(rc, "kv_dequant")
        return kd, vd

    def attend(self, query, num_heads, cos=None, sin=None, do_rotary=True, interleaved=False,
               scale=None, deq=None, layer_window=0, mask_window=0):
        """query [B, Sq, Hq*D] (pre-RoPE) over the cache; the last Sq tokens of each
        sequence are the query positions. layer_window: a sliding-window cache
        layer's last keys; mask_window: the GPU mask's window (<= 0: off).
        Returns [B, Sq, Hq*D] f32."""
        q = _f32(query)
        b, sq, _ = q.shape
        kd, vd = self.dequant() if deq is None else deq
        out = np.zeros_like(q)
        sl = np.ascontiguousarray(self.seq_len, dtype=np.int32)
        cosa = None if cos is None else _f32(cos)
        sina = None if sin is None else _f32(sin)
        rows = 0 if cosa is None else cosa.shape[0]
        rc = lib().sai_or_gqa_cached_window(
            _ptr(q), b, sq, num_heads, self.kv_heads, self.head_dim, _ptr(sl), self.t_cap,
            _ptr(kd), _ptr(vd), _ptr(cosa), _ptr(sina), rows, int(do_rotary), int(interleaved),
            int(scale is not None), 0.0 if scale is None else float(scale), int(layer_window),
            int(mask_window), _ptr(out))
        _check(rc, "gqa_cached")
        return out


def check_rhe_vs_rint(lo: int, hi: int) -> int:
    return int(lib().sai_or_check_rhe_vs_rint(lo, hi))
