"""Inputs and cases of the golden fixtures (test data, not product code).

Every input value comes from IEEE-exact or correctly rounded arithmetic on a
fixed integer stream, so a fixture regenerates bit for bit on any machine
(no libm transcendental, whose last bit may differ between hosts):

* integers: numpy's PCG64 bit generator seeded with [seed, stream], raw 64-bit
  outputs (the bit stream of a seeded bit generator is stable across numpy
  versions), read as little-endian 16-bit words;
* normals: Irwin-Hall, the sum of twelve uniforms (k + 0.5) / 65536 minus 6
  (mean 0, variance 1, range +-6); exact in f64, hence exact in f32;
* Student-t with 3 degrees of freedom: z / sqrt((z1^2 + z2^2 + z3^2) / 3), in
  f64 with one rounding per operation, then rounded to f32;
* bf16 inputs: round-to-nearest-even of the f32 values (integer arithmetic);
* RoPE tables: the rotation recurrence (c, s)[p+1] = (c, s)[p] * (cos t_i, sin t_i)
  in f64 from per-frequency steps (cos t_i, sin t_i) frozen in the manifest as
  hex floats, rounded to f32 once.

Seeds are 0x5A1A0000 + the workload's index (batch-1 decode 0, Llama layer 1,
int4 long context 2, prefill chunk 4).
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
MANIFEST = os.path.join(HERE, "manifest.json")
SEED_BASE = 0x5A1A0000
MAX_FIXTURE_BYTES = 64 * 1024
TAIL = 64  # tokens of stored codes at the end of each sequence

INT8, INT4 = 1, 2

# name -> case. appends: token counts appended (and committed) before the step
# under test. step: "decode" (separate append of one token, then decode),
# "fused" (append + decode in one launch) or "prefill" (append `new` tokens,
# then the prefill kernel). out_rows: query rows kept in the fixture.
CASES = {
    "decode_b1_8q2kv_d64_ctx512_int8": dict(
        cfg=0, batch=1, hq=8, hkv=2, d=64, theta=1e4, quant=INT8, q_dtype="f32",
        kv_dtype="f32", appends=[511], step="decode", new=1, k_dist="normal"),
    "decode_slice_4q1kv_d128_ctx8192_int8": dict(
        cfg=1, batch=1, hq=4, hkv=1, d=128, theta=5e5, quant=INT8, q_dtype="bf16",
        kv_dtype="f32", appends=[8128, 63], step="fused", new=1, k_dist="normal"),
    "decode_int4_outlier_4q1kv_d128_ctx4096": dict(
        cfg=2, batch=1, hq=4, hkv=1, d=128, theta=5e5, quant=INT4, q_dtype="bf16",
        kv_dtype="f32", appends=[4095], step="fused", new=1, k_dist="outlier_t3"),
    "prefill_4q1kv_d128_past192_new64_int8": dict(
        cfg=4, batch=1, hq=4, hkv=1, d=128, theta=5e5, quant=INT8, q_dtype="bf16",
        kv_dtype="bf16", appends=[192], step="prefill", new=64, k_dist="normal"),
}
OUTLIER_CHANNELS = (7, 31, 64, 100)


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def words16(seed: int, stream: int, n: int) -> np.ndarray:
    raw = np.random.PCG64([seed, stream]).random_raw((n + 3) // 4)
    return raw.astype("<u8").view("<u2")[:n]


def normals(seed: int, stream: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    u = words16(seed, stream, 12 * n).reshape(n, 12).astype(np.float64)
    z = ((u + 0.5) / 65536.0).sum(axis=1) - 6.0
    return z.astype(np.float32).reshape(shape)


def student_t3(seed: int, stream: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    z = normals(seed, stream, (4, n)).astype(np.float64)
    chi2 = z[1] * z[1] + z[2] * z[2] + z[3] * z[3]
    return (z[0] / np.sqrt(chi2 / 3.0)).astype(np.float32).reshape(shape)


def to_bf16_f32(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 (round to nearest even) -> f32, for finite inputs."""
    bits = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return bits.astype(np.uint32).view(np.float32)


def rope_steps(d: int, theta: float):
    """(cos t_i, sin t_i) for t_i = theta^(-2i/d): computed once by the
    fixture writer and frozen in the manifest."""
    t = theta ** (-(2.0 * np.arange(d // 2, dtype=np.float64)) / d)
    return np.cos(t), np.sin(t)


def rope_tables_from_steps(rows: int, cs: np.ndarray, sn: np.ndarray):
    c = np.ones_like(cs)
    s = np.zeros_like(sn)
    cos = np.empty((rows, cs.size), np.float64)
    sin = np.empty_like(cos)
    for p in range(rows):
        cos[p], sin[p] = c, s
        c, s = c * cs - s * sn, s * cs + c * sn
    return cos.astype(np.float32), sin.astype(np.float32)


def load_manifest() -> dict:
    with open(MANIFEST) as f:
        return json.load(f)


def rope_for(name: str, manifest: dict | None = None):
    """RoPE tables of a case, from the steps frozen in the manifest."""
    c = CASES[name]
    m = (manifest or load_manifest())[name]["rope"]
    cs = np.array([float.fromhex(h) for h in m["cos_step_hex"]])
    sn = np.array([float.fromhex(h) for h in m["sin_step_hex"]])
    assert cs.size == c["d"] // 2
    return rope_tables_from_steps(m["rows"], cs, sn)


def total_tokens(name: str) -> int:
    c = CASES[name]
    return sum(c["appends"]) + c["new"]


def inputs(name: str):
    """(appends, step_kv, q): appends is a list of (k, v) [B, n, Hkv*D] f32 for
    the committed prefix, step_kv the step's (k, v), q [B, new, Hq*D] f32; bf16
    inputs are already rounded to bf16 values."""
    c = CASES[name]
    seed = SEED_BASE + c["cfg"]
    b, hkv, hq, d = c["batch"], c["hkv"], c["hq"], c["d"]

    def kv(i, n):
        shape = (b, n, hkv * d)
        if c["k_dist"] == "outlier_t3":
            k = student_t3(seed, 10 + i, shape).reshape(b, n, hkv, d)
            k[..., list(OUTLIER_CHANNELS)] *= np.float32(20.0)
            k = k.reshape(shape)
        else:
            k = normals(seed, 10 + i, shape)
        v = normals(seed, 20 + i, shape)
        if c["kv_dtype"] == "bf16":
            k, v = to_bf16_f32(k), to_bf16_f32(v)
        return k, v

    appends = [kv(i, n) for i, n in enumerate(c["appends"])]
    step = kv(len(c["appends"]), c["new"])
    q = normals(seed, 30, (b, c["new"], hq * d))
    if c["q_dtype"] == "bf16":
        q = to_bf16_f32(q)
    return appends, step, q


def out_rows(name: str):
    """Query rows kept in the fixture: all for a decode step; for the prefill
    chunk every fourth row and the last (the full output would exceed the
    fixture size)."""
    c = CASES[name]
    n = c["new"]
    if n == 1:
        return np.array([0])
    return np.unique(np.concatenate([np.arange(0, n, 4), [n - 1]]))


def cache_arrays(codes_k, codes_v, params_k, params_v, n):
    """The cache contents over tokens [0, n) as one dict of arrays."""
    return {"k_codes": codes_k[:, :, :n], "v_codes": codes_v[:, :, :n],
            "k_params": params_k[:, :, :n], "v_params": params_v[:, :, :n]}


def tails(arrays: dict, n: int) -> dict:
    t0 = max(0, n - TAIL)
    return {f"{k}_tail": np.ascontiguousarray(v[:, :, t0:n]) for k, v in arrays.items()}


def oracle_run(name: str, manifest: dict | None = None):
    """The oracle's cache contents (tokens [0, total)) and kept output rows."""
    import oracle as O
    c = CASES[name]
    cos, sin = rope_for(name, manifest)
    appends, (ks, vs), q = inputs(name)
    t = total_tokens(name)
    oc = O.LogicalCache(c["batch"], c["hkv"], c["d"], t, c["quant"])
    for k, v in appends:
        oc.append(k, v, cos, sin)
    oc.append(ks, vs, cos, sin)
    out = oc.attend(q, c["hq"], cos, sin)
    if c["quant"] == INT8:
        kp, vp = oc.k_scale, oc.v_scale
    else:
        kp, vp = oc.k_sz, oc.v_sz
    return cache_arrays(oc.k_codes, oc.v_codes, kp, vp, t), out[:, out_rows(name)]


def load_fixture(name: str, manifest: dict | None = None) -> dict:
    m = (manifest or load_manifest())[name]
    with np.load(os.path.join(HERE, m["file"]), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}
