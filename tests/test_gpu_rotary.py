"""GPU parity of the standalone RotaryEmbedding kernel and of the RoPE table
generator, through the C ABI (sai_rotary_embedding, sai_rope_tables).

Bar: bit-exact. The rotation is two rounded f32 products and one rounded
add/sub per element, as apply_rope_in_place (onnx-rt/src/ops/microsoft.rs:177-233)
computes it; the oracle's apply_rope restates that function, and bf16 outputs
are the oracle's f32 result rounded to nearest even. The tables are the
Gemma loader's precompute (model_loader/gemma.rs:458-541), restated by the
oracle op for op.

Also restated: the reference's GPU rotary tests (onnx-rt/tests/test_cuda.rs:
2622-2830: small split-half f32, decode-step interleaved, bf16 Gemma shape
against the CPU op, odd head_dim rejected).
"""
import numpy as np
import pytest

import oracle as O
import smallaios_amd as S
from _gpu_util import log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    assert S.lib().sai_device_supported(0) == 1, "device 0 is not gfx950"
    r = S.Runtime(0)
    yield r
    r.close()


def tables_f32(rows, half, theta=10000.0):
    """f64 angles rounded once to f32 (any table works: both sides read it)."""
    inv = theta ** (-(2.0 * np.arange(half)) / (2 * half))
    ang = np.arange(rows, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def to_dev(a: np.ndarray, bf16: bool, offset: int = 0):
    """Device copy; bf16 from the exact bits of O.f32_to_bf16_bits. offset:
    elements of padding in front (to make a pointer that is not 16-byte
    aligned)."""
    import torch
    if bf16:
        bits = O.f32_to_bf16_bits(a).ravel()
        buf = torch.zeros(bits.size + offset, dtype=torch.int16)
        buf[offset:] = torch.from_numpy(bits.view(np.int16))
        return buf.cuda().view(torch.bfloat16)[offset:]
    buf = torch.zeros(a.size + offset, dtype=torch.float32)
    buf[offset:] = torch.from_numpy(np.ascontiguousarray(a, np.float32).ravel())
    return buf.cuda()[offset:]


def from_dev(t, bf16: bool) -> np.ndarray:
    import torch
    if bf16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def oracle_rope(x, b, h, s, d, layout, cos, sin, ids, interleaved, rotary_dim):
    """Oracle over the same rows: x flat in the given layout."""
    rotary_dim = rotary_dim if rotary_dim > 0 else None
    if layout == S.ROPE_BHSD:
        return O.apply_rope(x.reshape(b, h, s, d), cos, sin, ids, interleaved,
                            rotary_dim).ravel()
    v = x.reshape(b, s, h, d).transpose(0, 2, 1, 3)
    out = O.apply_rope(v, cos, sin, ids, interleaved, rotary_dim)
    return out.transpose(0, 2, 1, 3).ravel()


def run_case(rt, *, b, h, s, d, layout=S.ROPE_BHSD, dtype="f32", table="f32", interleaved=False,
             rotary_dim=0, pos_mode="start", start=0, rows=None, inplace=False, offset=0,
             seed=0):
    rng = np.random.default_rng(seed)
    rd = d if rotary_dim <= 0 else rotary_dim
    half = rd // 2
    if pos_mode == "start":
        ids_host = None
        ids = np.arange(s) + start
    elif pos_mode == "shared_affine":
        ids_host = np.arange(s) + start
        ids = ids_host
    elif pos_mode == "shared":
        ids_host = rng.integers(0, (rows or 64), size=s)
        ids = ids_host
    elif pos_mode == "per_row_affine":
        starts = rng.integers(0, 40, size=b)
        ids_host = (starts[:, None] + np.arange(s)[None, :]).ravel()
        ids = ids_host
    else:  # per_row
        ids_host = rng.integers(0, (rows or 64), size=b * s)
        ids = ids_host
    rows = rows or int(np.max(ids)) + 1 + 3
    cos, sin = tables_f32(rows, half)
    x = rng.standard_normal(b * h * s * d).astype(np.float32) * 3
    xb = dtype == "bf16"
    tb = table == "bf16"
    if xb:
        x = O.bf16_bits_to_f32(O.f32_to_bf16_bits(x))
    if tb:
        cos = O.bf16_bits_to_f32(O.f32_to_bf16_bits(cos))
        sin = O.bf16_bits_to_f32(O.f32_to_bf16_bits(sin))
    xd = to_dev(x, xb, offset)
    yd = xd if inplace else to_dev(np.full_like(x, 7.0), xb, offset)
    cd = to_dev(cos, tb).reshape(rows, half)
    sd = to_dev(sin, tb).reshape(rows, half)
    rt.rotary_embedding(xd, yd, b, h, s, d, cd, sd, position_ids=ids_host, start_position=start,
                        layout=layout, rotary_dim=rotary_dim, interleaved=interleaved,
                        dtype=S.DTYPE_BF16 if xb else S.DTYPE_F32,
                        table_dtype=S.DTYPE_BF16 if tb else S.DTYPE_F32)
    import torch
    torch.cuda.synchronize()
    got = from_dev(yd, xb)
    want = oracle_rope(x, b, h, s, d, layout, cos, sin, ids, interleaved, rotary_dim)
    if xb:
        want = O.f32_to_bf16_bits(want)
        assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]
    else:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
            np.flatnonzero(got != want)[:10]


CASES = []
_rng = np.random.default_rng(0x5A1A)
for _i in range(40):
    CASES.append(dict(
        b=int(_rng.integers(1, 4)), h=int(_rng.integers(1, 5)), s=int(_rng.integers(1, 9)),
        d=int(_rng.choice([128, 64, 6, 32, 10])),
        layout=int(_rng.integers(0, 2)), dtype=str(_rng.choice(["f32", "bf16"])),
        table=str(_rng.choice(["f32", "bf16"])), interleaved=bool(_rng.integers(0, 2)),
        partial=bool(_rng.integers(0, 3) == 0),
        pos_mode=str(_rng.choice(["start", "shared_affine", "shared", "per_row_affine",
                                  "per_row"])),
        start=int(_rng.integers(0, 30)), inplace=bool(_rng.integers(0, 2)),
        offset=int(_rng.choice([0, 0, 1])), seed=_i))


@pytest.mark.parametrize("c", CASES, ids=[f"case{i}" for i in range(len(CASES))])
def test_rotary_matrix_bit_exact(rt, c):
    c = dict(c)
    partial = c.pop("partial")
    d = c["d"]
    c["rotary_dim"] = (d // 2 if (d // 2) % 2 == 0 else d - 2) if partial else 0
    log(f"rotary {c}")
    run_case(rt, **c)


@pytest.mark.parametrize("kw", [
    # more than one launch: sequence chunks of explicit positions
    dict(b=2, h=2, s=1200, d=64, pos_mode="shared", rows=4096),
    dict(b=3, h=1, s=700, d=128, pos_mode="per_row", rows=2048, dtype="bf16"),
    # more than 512 sequences with one start each
    dict(b=600, h=1, s=3, d=32, pos_mode="per_row_affine"),
    dict(b=700, h=2, s=2, d=64, pos_mode="start", start=5, layout=S.ROPE_BSHD),
    # a Llama-sized prefill chunk, in place
    dict(b=1, h=32, s=512, d=128, pos_mode="shared_affine", start=100, inplace=True,
         dtype="bf16", table="bf16"),
])
def test_rotary_chunked_launches(rt, kw):
    log(f"rotary chunked {kw}")
    run_case(rt, seed=11, **kw)


# -------------------------------------------- reference GPU tests restated ---
def test_reference_small_split_half_f32(rt):
    # test_cuda.rs:2622-2665: [1, 2, 4, 8], position 0, x = i * 0.0125 - 0.25
    import torch
    b, h, s, d = 1, 2, 4, 8
    x = (np.arange(b * h * s * d, dtype=np.float32) * np.float32(0.0125)
         - np.float32(0.25)).astype(np.float32)
    cos, sin = tables_f32(16, d // 2)
    xd, yd = to_dev(x, False), to_dev(np.zeros_like(x), False)
    rt.rotary_embedding(xd, yd, b, h, s, d, to_dev(cos, False).reshape(16, 4),
                        to_dev(sin, False).reshape(16, 4), start_position=0)
    torch.cuda.synchronize()
    got = from_dev(yd, False)
    want = O.apply_rope(x.reshape(b, h, s, d), cos, sin, np.arange(s)).ravel()
    assert np.array_equal(got, want)
    assert np.abs(got - want).max() < 1e-5


def test_reference_decode_step_interleaved(rt):
    # test_cuda.rs:2667-2707: [2, 4, 1, 16], position 37, interleaved
    import torch
    b, h, s, d = 2, 4, 1, 16
    x = np.sin(np.arange(b * h * s * d, dtype=np.float32) * np.float32(0.07)).astype(np.float32)
    cos, sin = tables_f32(64, d // 2)
    xd, yd = to_dev(x, False), to_dev(np.zeros_like(x), False)
    rt.rotary_embedding(xd, yd, b, h, s, d, to_dev(cos, False).reshape(64, 8),
                        to_dev(sin, False).reshape(64, 8), start_position=37, interleaved=True)
    torch.cuda.synchronize()
    want = O.apply_rope(x.reshape(b, h, s, d), cos, sin, [37], interleaved=True).ravel()
    assert np.array_equal(from_dev(yd, False), want)


def test_reference_bf16_gemma_shape(rt):
    # test_cuda.rs:2709-2805: [1, 8, 8, 128] bf16, position 0, against the
    # f32 CPU op on the bf16-rounded input within 1e-2 (and bit-exact after
    # rounding the CPU result)
    import torch
    b, h, s, d = 1, 8, 8, 128
    x = (np.cos(np.arange(b * h * s * d, dtype=np.float32) * np.float32(0.001))
         * np.float32(0.5)).astype(np.float32)
    xr = O.bf16_bits_to_f32(O.f32_to_bf16_bits(x))
    cos, sin = tables_f32(32, d // 2)
    xd = to_dev(x, True)
    yd = to_dev(np.zeros_like(x), True)
    rt.rotary_embedding(xd, yd, b, h, s, d, to_dev(cos, False).reshape(32, 64),
                        to_dev(sin, False).reshape(32, 64), start_position=0)
    torch.cuda.synchronize()
    got = O.bf16_bits_to_f32(from_dev(yd, True))
    cpu = O.apply_rope(xr.reshape(b, h, s, d), cos, sin, np.arange(s)).ravel()
    assert np.abs(got - cpu).max() < 1e-2
    assert np.array_equal(from_dev(yd, True), O.f32_to_bf16_bits(cpu))


def test_errors_leave_output_untouched(rt):
    import torch
    b, h, s, d = 1, 2, 3, 8
    cos, sin = tables_f32(8, 4)
    cd, sd = to_dev(cos, False).reshape(8, 4), to_dev(sin, False).reshape(8, 4)
    x = to_dev(np.ones(b * h * s * d, np.float32), False)
    y = to_dev(np.full(b * h * s * d, 5.0, np.float32), False)

    def call(**kw):
        args = dict(position_ids=None, start_position=0, layout=S.ROPE_BHSD, rotary_dim=0,
                    interleaved=False)
        args.update(kw)
        dd = args.pop("d", d)
        with pytest.raises(S.SaiError) as e:
            rt.rotary_embedding(x, y, b, h, s, dd, args.pop("cos", cd), args.pop("sin", sd),
                                **args)
        return e.value

    e = call(position_ids=[0, 1])  # length neither Sq nor B*Sq
    assert e.kind == "ShapeMismatch" and "position_ids length 2 != B*Sq = 3" in str(e)
    e = call(position_ids=[0, 1, 8])
    assert e.kind == "ShapeMismatch" and "position 8 out of cache range 8" in str(e)
    e = call(position_ids=[0, -1, 2])
    assert "position -1 out of cache range 8" in str(e)
    e = call(start_position=6)  # 6 + 3 > 8
    assert e.kind == "ShapeMismatch" and "exceeds cos/sin table length" in str(e)
    e = call(rotary_dim=10)
    assert e.kind == "InvalidAttribute" and "rotary_dim must be in 1..=head_dim" in str(e)
    e = call(rotary_dim=6)
    assert e.kind == "ShapeMismatch" and "cache inner dim 4 != rotary_dim/2 = 3" in str(e)
    e = call(d=7, rotary_dim=0)  # odd head_dim (test_cuda.rs:2807-2830)
    assert e.kind == "InvalidAttribute" and "rotary_dim must be even" in str(e)
    e = call(layout=2)
    assert e.kind == "InvalidAttribute"
    st = S.lib().sai_rotary_embedding(rt.handle, S._dev_ptr(x), S._dev_ptr(y), 10, b, h, s, d, 0,
                                      None, 0, 0, S._dev_ptr(cd), S._dev_ptr(sd), 1, 8, 4, 0, 0,
                                      None)
    assert st == -3  # F16 input is not supported
    st = S.lib().sai_rotary_embedding(rt.handle, S._dev_ptr(x), S._dev_ptr(y), 1, b, h, s, d, 0,
                                      None, 0, 0, None, S._dev_ptr(sd), 1, 8, 4, 0, 0, None)
    assert st == -2 and "missing cos_cache" in rt.last_error()
    torch.cuda.synchronize()
    assert np.all(from_dev(y, False) == 5.0)
    # zero rows: nothing to do, no error
    rt.rotary_embedding(x, y, 0, h, s, d, cd, sd, start_position=0)
    rt.rotary_embedding(x, y, b, 0, s, d, cd, sd, position_ids=[0, 1, 99])  # no rows, no check
    torch.cuda.synchronize()
    assert np.all(from_dev(y, False) == 5.0)


# ------------------------------------------------------------------ tables ---
@pytest.mark.parametrize("max_pos,half,theta", [
    (8192, 64, 10_000.0), (4096, 128, 1_000_000.0), (131072, 128, 500_000.0), (33, 3, 5e5),
    (1, 1, 10_000.0)])
def test_rope_tables_bit_exact(rt, max_pos, half, theta):
    import torch
    log(f"rope tables {max_pos}x{half} theta {theta}")
    want_c, want_s = O.rope_tables_bf16(max_pos, half, theta)
    c = torch.empty(max_pos * half, dtype=torch.int16, device="cuda")
    s = torch.empty_like(c)
    rt.rope_tables(max_pos, half, theta, c, s, dtype=S.DTYPE_BF16)
    cf = torch.empty(max_pos * half, dtype=torch.float32, device="cuda")
    sf = torch.empty_like(cf)
    rt.rope_tables(max_pos, half, theta, cf, sf, dtype=S.DTYPE_F32)
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy().view(np.uint16), want_c.ravel())
    assert np.array_equal(s.cpu().numpy().view(np.uint16), want_s.ravel())
    assert np.array_equal(cf.cpu().numpy(), O.bf16_bits_to_f32(want_c).ravel())
    assert np.array_equal(sf.cpu().numpy(), O.bf16_bits_to_f32(want_s).ravel())


def test_generated_bf16_tables_drive_the_rotation(rt):
    """The loader's bf16 tables fed straight to the rotation (read as their
    exact f32 values) give what the f32 cast of them gives."""
    import torch
    max_pos, half = 256, 64
    c = torch.empty(max_pos, half, dtype=torch.bfloat16, device="cuda")
    s = torch.empty_like(c)
    rt.rope_tables(max_pos, half, 1e6, c, s, dtype=S.DTYPE_BF16)
    cf, sf = c.float(), s.float()
    rng = np.random.default_rng(5)
    x = rng.standard_normal(2 * 4 * 16 * 128).astype(np.float32)
    xd = to_dev(x, False)
    y1 = torch.empty_like(xd)
    y2 = torch.empty_like(xd)
    rt.rotary_embedding(xd, y1, 2, 4, 16, 128, c, s, start_position=200)
    rt.rotary_embedding(xd, y2, 2, 4, 16, 128, cf, sf, start_position=200)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    want = O.apply_rope(x.reshape(2, 4, 16, 128), cf.cpu().numpy(), sf.cpu().numpy(),
                        np.arange(200, 216)).ravel()
    assert np.array_equal(y1.cpu().numpy(), want)


def test_rotary_bf16_rounding_patterns(rt):
    """bf16 outputs round like the reference's f32_to_bf16 (tensor.rs:312-329) on every
    kind of f32 the rotation can produce: with x = 1 and sin = 0 each output is its cos
    entry, so the f32 table carries the patterns (262,144 of them): every exponent from
    denormals to the largest finite binade, low halves exactly at a tie (0x8000, with
    the kept bit odd and even), one below and above it, 0x0000, 0xFFFF and random, and
    both signs. (NaN is not among them: a NaN's payload after the rotation's arithmetic
    is the device's, not the rounding's.)"""
    import torch
    rng = np.random.default_rng(0xBF16)
    s, d = 4096, 128
    half = d // 2
    n = s * half
    sign = rng.integers(0, 2, n, dtype=np.uint32) << 31
    expo = (np.arange(n, dtype=np.uint32) % 255) << 23
    high = rng.integers(0, 128, n, dtype=np.uint32) << 16
    lows = np.array([0x8000, 0x8000, 0x7FFF, 0x8001, 0x0000, 0xFFFF], np.uint32)
    pick = rng.integers(0, len(lows) + 2, n)
    low = np.where(pick < len(lows), lows[np.minimum(pick, len(lows) - 1)],
                   rng.integers(0, 1 << 16, n, dtype=np.uint32))
    # the kept bit (bit 16) odd for half of the exact ties
    high = np.where((pick == 1), high | (1 << 16), high)
    cos = (sign | expo | high | low).view(np.float32).reshape(s, half)
    sin = np.zeros_like(cos)
    x = np.ones(s * d, np.float32)
    xd = to_dev(x, True)
    yd = to_dev(np.zeros_like(x), True)
    cd = to_dev(cos, False).reshape(s, half)
    sd = to_dev(sin, False).reshape(s, half)
    log("rotary bf16 rounding: 262,144 f32 patterns through the output conversion")
    rt.rotary_embedding(xd, yd, 1, 1, s, d, cd, sd, start_position=0, layout=S.ROPE_BSHD,
                        dtype=S.DTYPE_BF16, table_dtype=S.DTYPE_F32)
    torch.cuda.synchronize()
    got = from_dev(yd, True)
    y = oracle_rope(x, 1, 1, s, d, S.ROPE_BSHD, cos, sin, np.arange(s), False, 0)
    want = O.f32_to_bf16_bits(y)
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]
    # the patterns reach the conversion unchanged: the first half of each row is
    # cos - 0 = cos, bit for bit
    assert np.array_equal(y.reshape(s, d)[:, :half].view(np.uint32), cos.view(np.uint32))
