"""Pins the CPU oracle (oracle/sai_oracle.c) before it is trusted as the checker.

How each oracle function is pinned (none of them is checked by retyping its
own formula):

* expf_approx (operators.rs:1328-1357): exact at x = 0, the clamp/underflow
  rules, and the bound |e^x - approx| <= 7e-5 relative that the degree-4
  Taylor remainder (|f| <= ln2/2) implies -- a dropped or wrong term breaks it by >100x.
* round_half_even (quantized.rs:33-50): the reference's QuantizeLinear
  known answers (quantized.rs:422-449) and an exhaustive proof over all 2^32
  f32 bit patterns that the int8 code it yields equals the one from IEEE
  roundTiesToEven (rintf), which is what the HIP kernel uses.
* sqrt_f32 / default scale (microsoft.rs:54-63, :1153): equals
  1/sqrt(D) to 1 ulp for the head dims of the path.
* f32 -> binary16 (int4 scale/zero storage): exhaustive over every f32 with
  exponent in the binary16 range and all specials against numpy's float16
  conversion (IEEE RNE).
* f32_to_bf16 (tensor.rs:312-329): tie patterns against torch's bf16 RNE.
* pack_bits/unpack_bits (kv_compression.rs:294-333): the reference's round
  trips (kv_compression.rs:1195-1216) and hand-derived LSB-first bytes.
* RoPE (microsoft.rs:177-233): the reference's KATs rope_position_zero_is_identity
  and rope_non_interleaved_manual_calc (microsoft.rs:1346, :1381) with its
  Taylor tables, interleaved-differs, and a vectorised numpy float32
  restatement (bit-exact: numpy float32 multiply/subtract are single IEEE ops).
* SDPA / GQA (microsoft.rs:380-438, :1082-1190): the reference's KATs at
  microsoft.rs:1421, 1461, 1490, 1941, 1951, 1976 and its GQA error/shape tests
  (1602-1824, 2032-2177), plus f64 brute-force attention on random inputs.
* int8 / int4 KV quantisers (composed spec, no reference implementation):
  an independent vectorised numpy restatement using np.rint / np.float16,
  plus invariants (|code| <= 127, a +-127 code at every row maximum, error <=
  s/2 per element; int4 codes in [0, 15], error <= s/2 + f16 rounding).
"""
import math
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle as O

f32 = np.float32


# ------------------------------------------------------------ expf_approx ---
def test_expf_approx_structure():
    assert O.expf_approx(np.array([0.0], f32))[0] == 1.0
    # x = k*ln2 exactly representable multiples give 2^k up to the tail error
    x = np.linspace(-20, 20, 200001, dtype=f32)
    got = O.expf_approx(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    rel = np.abs(got - ref) / ref
    # Taylor remainder |f|^5/120 / e^f at f = -ln2/2 is 6.3e-5; a dropped f^4
    # term costs 8.5e-4, a wrong sign on any term more
    assert rel.max() < 7e-5, rel.max()
    assert rel.max() > 1e-6
    # clamp to -88.7, then k = -128 trips the underflow rule (k + 127 < 0 -> 0)
    assert O.expf_approx(np.array([-100.0, -88.7], f32)).tolist() == [0.0, 0.0]
    assert O.expf_approx(np.array([-87.0], f32))[0] > 0


# -------------------------------------------------------- round_half_even ---
def test_quantize_linear_known_answers():
    # quantized.rs:422-429 / 442-449 (scale 0.1, zp 0)
    for xs, want in [([0.0, 0.1, 0.2, -0.1], [0, 1, 2, -1]), ([100.0, -100.0], [127, -128])]:
        x = np.array(xs, f32) / f32(0.1)
        r = O.round_half_even(x)
        codes = np.clip(r, -128, 127).astype(np.int32)
        assert codes.tolist() == want


def test_round_half_even_ties():
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 1e8 + 1, -0.49999997], f32)
    assert O.round_half_even(x).tolist() == np.rint(x).tolist()


@pytest.mark.slow
def test_round_half_even_int8_code_exhaustive():
    """All 2^32 f32 patterns: clamp(sat_i32(rhe(x))) == clamp(sat_i32(rint(x)))."""
    chunks = [(i << 28, (i + 1) << 28) for i in range(16)]
    with ThreadPoolExecutor(8) as ex:
        bad = sum(ex.map(lambda c: O.check_rhe_vs_rint(*c), chunks))
    assert bad == 0


# ----------------------------------------------------------- sqrt / scale ---
@pytest.mark.parametrize("d", [2, 4, 64, 128, 256])
def test_default_scale(d):
    s = O.default_scale(d)
    assert abs(s - 1 / math.sqrt(d)) <= 2 * np.spacing(f32(s))


# ------------------------------------------------------------------- f16 ---
@pytest.mark.slow
def test_f16_rne_against_numpy_exhaustive_range():
    chunk = 1 << 23
    for exp in range(100, 145):  # every f32 whose magnitude matters for binary16
        base = np.uint32(exp << 23)
        u = (np.arange(chunk, dtype=np.uint32) + base)
        for sign in (0, 0x80000000):
            x = (u | np.uint32(sign)).view(f32)
            with np.errstate(over="ignore"):  # values past 65520 round to inf, as intended
                want = x.astype(np.float16).view(np.uint16)
            np.testing.assert_array_equal(O.f32_to_f16_bits(x), want)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 1e-8, 3e-8,
                        6e-8, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25, 2.0 ** -26, 1e-30, 1e38],
                       f32)
    with np.errstate(over="ignore"):
        want = special.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(O.f32_to_f16_bits(special), want)


def test_f16_roundtrip_small():
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    x = h.view(np.float16).astype(f32)
    np.testing.assert_array_equal(O.f32_to_f16_bits(x), h)


def test_bf16_ties_against_torch():
    torch = pytest.importorskip("torch")
    u = np.array([0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F807FFF, 0x7F7FFFFF, 0xFF800000,
                  0x00008000, 0x80018000], dtype=np.uint32)
    x = u.view(f32)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.f32_to_bf16_bits(x), want)


# --------------------------------------------------------------- packing ---
def test_pack_bits_reference_roundtrips():
    for vals, bits in [(list(range(16)), 4), ([0, 1, 2, 3, 4, 5, 6, 7, 0, 3, 5, 7], 3),
                       (list(range(255)), 8)]:
        p = O.pack_bits(vals, bits)
        assert O.unpack_bits(p, len(vals), bits).tolist() == vals


def test_pack_bits_lsb_first_bytes():
    # element 2i in the low nibble of byte i
    assert O.pack_bits([1, 2, 3, 4], 4).tolist() == [0x21, 0x43]
    assert O.pack_bits([0xF, 0x0, 0x0, 0xF], 4).tolist() == [0x0F, 0xF0]


# ------------------------------------------------------------------ RoPE ---
def _taylor_tables(max_seq, half):
    # make_rope_caches of microsoft.rs:1318-1343 (f32 throughout)
    cos = np.zeros((max_seq, half), f32)
    sin = np.zeros((max_seq, half), f32)
    for p in range(max_seq):
        for i in range(half):
            th = f32(p) * (f32(0.1) + f32(i) * f32(0.01))
            x2 = th * th
            cos[p, i] = f32(1.0) - x2 / f32(2.0) + x2 * x2 / f32(24.0) - x2 * x2 * x2 / f32(720.0)
            sin[p, i] = th * (f32(1.0) - x2 / f32(6.0) + x2 * x2 / f32(120.0)
                              - x2 * x2 * x2 / f32(5040.0))
    return cos, sin


def test_rope_position_zero_is_identity():
    cos, sin = _taylor_tables(4, 2)
    x = np.array([1, 2, 3, 4], f32).reshape(1, 1, 1, 4)
    np.testing.assert_allclose(O.apply_rope(x, cos, sin, [0]).ravel(), [1, 2, 3, 4], atol=1e-5)


def test_rope_non_interleaved_manual_calc():
    cos, sin = _taylor_tables(2, 2)
    x = np.array([1, 2, 3, 4], f32).reshape(1, 1, 1, 4)
    v = O.apply_rope(x, cos, sin, [1]).ravel()
    c0, s0, c1, s1 = cos[1, 0], sin[1, 0], cos[1, 1], sin[1, 1]
    want = [c0 * 1 - s0 * 3, c1 * 2 - s1 * 4, s0 * 1 + c0 * 3, s1 * 2 + c1 * 4]
    np.testing.assert_allclose(v, want, atol=1e-4)


def test_rope_interleaved_differs_and_errors():
    cos, sin = _taylor_tables(4, 2)
    x = np.array([1, 2, 3, 4], f32).reshape(1, 1, 1, 4)
    a = O.apply_rope(x, cos, sin, [1], interleaved=False)
    b = O.apply_rope(x, cos, sin, [1], interleaved=True)
    assert np.abs(a - b).max() > 1e-4
    with pytest.raises(O.OracleError):
        O.apply_rope(x, cos, sin, [4])  # position out of cache range
    with pytest.raises(O.OracleError):
        O.apply_rope(x, cos[:, :1], sin[:, :1], [0])  # cache inner dim != D/2


@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_matches_vectorised_float32(interleaved):
    import smallaios_amd as S
    rng = np.random.default_rng(3)
    b, h, sq, d = 2, 3, 5, 64
    x = rng.standard_normal((b, h, sq, d)).astype(f32)
    cos, sin = S.rope_tables(64, d, 10000.0)
    pos = np.arange(sq) + 7
    got = O.apply_rope(x, cos, sin, pos, interleaved=interleaved)
    c = cos[pos][None, None]
    s = sin[pos][None, None]
    if interleaved:
        x0, x1 = x[..., 0::2], x[..., 1::2]
    else:
        x0, x1 = x[..., : d // 2], x[..., d // 2:]
    y0 = c * x0 - s * x1
    y1 = s * x0 + c * x1
    want = np.empty_like(x)
    if interleaved:
        want[..., 0::2], want[..., 1::2] = y0, y1
    else:
        want[..., : d // 2], want[..., d // 2:] = y0, y1
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------------- SDPA ---
def test_sdpa_single_head_non_causal_matches_manual():
    q = np.array([1, 0], f32).reshape(1, 1, 1, 2)
    k = np.array([1, 0, 0, 1], f32).reshape(1, 1, 2, 2)
    v = np.array([1, 2, 3, 4], f32).reshape(1, 1, 2, 2)
    out = O.sdpa(q, k, v, 1, 0, 1.0, False).ravel()
    e = O.expf_approx(np.array([1.0], f32))[0]
    s0, s1 = e / (e + 1), 1 / (e + 1)
    np.testing.assert_allclose(out, [s0 + 3 * s1, 2 * s0 + 4 * s1], atol=1e-4)


def test_sdpa_causal_mask_exact_zero():
    q = np.ones((1, 1, 3, 1), f32)
    v = np.array([2, 4, 8], f32).reshape(1, 1, 3, 1)
    out = O.sdpa(q, q, v, 1, 0, 1.0, True).ravel()
    np.testing.assert_allclose(out, [2, 3, 14 / 3], atol=1e-3)


def test_sdpa_gqa_grouping():
    q = np.zeros((1, 2, 1, 2), f32)
    k = np.array([1, 0, 0, 1], f32).reshape(1, 1, 2, 2)
    v = np.array([2, 3, 4, 5], f32).reshape(1, 1, 2, 2)
    out = O.sdpa(q, k, v, 1, 0, 1.0, False).reshape(2, 2)
    np.testing.assert_allclose(out, [[3, 4], [3, 4]], atol=1e-4)


def test_sdpa_empty_keys_and_causal_windows():
    q = np.array([1, 2], f32).reshape(1, 1, 1, 2)
    e = np.zeros((1, 1, 0, 2), f32)
    assert O.sdpa(q, e, e, 1, 0, 1.0, False).ravel().tolist() == [0.0, 0.0]
    q1 = np.ones((1, 1, 1, 1), f32)
    k = np.array([10, 20, 30, 40], f32).reshape(1, 1, 4, 1)
    v = np.array([1, 2, 3, 4], f32).reshape(1, 1, 4, 1)
    assert abs(O.sdpa(q1, k, v, 1, 0, 1.0, True).ravel()[0] - 1.0) < 1e-5
    k1 = np.ones((1, 1, 4, 1), f32)
    assert abs(O.sdpa(q1, k1, v, 1, 2, 1.0, True).ravel()[0] - 2.0) < 1e-3
    with pytest.raises(O.OracleError):
        O.sdpa(np.zeros((1, 3, 1, 2), f32), np.zeros((1, 2, 1, 2), f32),
               np.zeros((1, 2, 1, 2), f32), 2, 0, 1.0, False)


def test_sdpa_matches_f64_bruteforce():
    rng = np.random.default_rng(5)
    b, hq, hk, sq, sk, d, past = 2, 8, 2, 3, 40, 16, 37
    q = rng.standard_normal((b, hq, sq, d)).astype(f32)
    k = rng.standard_normal((b, hk, sk, d)).astype(f32)
    v = rng.standard_normal((b, hk, sk, d)).astype(f32)
    got = O.sdpa(q, k, v, hk, past, 0.25, True)
    g = hq // hk
    for bi in range(b):
        for h in range(hq):
            kk = k[bi, h // g].astype(np.float64)
            vv = v[bi, h // g].astype(np.float64)
            for i in range(sq):
                s = kk @ q[bi, h, i].astype(np.float64) * 0.25
                s[past + i + 1:] = -np.inf
                p = np.exp(s - s.max())
                want = (p / p.sum()) @ vv
                np.testing.assert_allclose(got[bi, h, i], want, atol=2e-5, rtol=1e-4)


# -------------------------------------------------------------------- GQA ---
def _gqa_inputs(sq=1, q_hidden=8, kv_hidden=4, v_hidden=None):
    q = np.zeros((1, sq, q_hidden), f32)
    k = np.zeros((1, sq, kv_hidden), f32)
    v = np.zeros((1, sq, v_hidden or kv_hidden), f32)
    return q, k, v


def test_gqa_shapes_and_cache_growth():
    q, k, v = _gqa_inputs()
    k[:] = [1, 0, 0, 1]
    v[:] = [1, 2, 3, 4]
    a, pk, pv = O.gqa(q, k, v, 4, 2, do_rotary=False)
    assert a.shape == (1, 1, 8) and pk.shape == (1, 2, 1, 2) and pv.shape == (1, 2, 1, 2)
    q1, k1, v1 = np.zeros((1, 2, 8), f32), np.ones((1, 2, 4), f32), 2 * np.ones((1, 2, 4), f32)
    _, pk1, pv1 = O.gqa(q1, k1, v1, 4, 2, do_rotary=False)
    assert pk1.shape == (1, 2, 2, 2)
    _, pk2, _ = O.gqa(np.zeros((1, 1, 8), f32), 3 * np.ones((1, 1, 4), f32),
                      4 * np.ones((1, 1, 4), f32), 4, 2, pk1, pv1, do_rotary=False)
    assert pk2.shape == (1, 2, 3, 2)
    q3, k3, v3 = np.zeros((1, 2, 8), f32), np.zeros((1, 2, 4), f32), np.zeros((1, 2, 4), f32)
    _, pk3, pv3 = O.gqa(q3, k3, v3, 4, 2, np.zeros((1, 2, 3, 2), f32), np.zeros((1, 2, 3, 2), f32),
                        do_rotary=False)
    assert pk3.shape == (1, 2, 5, 2) and pv3.shape == (1, 2, 5, 2)


def test_gqa_errors():
    q, k, v = _gqa_inputs()
    with pytest.raises(O.OracleError) as e:
        O.gqa(q, k, v, 4, 2, do_rotary=True)  # no cos/sin
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(O.OracleError) as e:
        O.gqa(q, k, v, 4, 2, local_window_size=512, do_rotary=False)
    assert e.value.kind == "InvalidAttribute"
    for nh, kvh in [(0, 2), (4, 0), (3, 2)]:
        with pytest.raises(O.OracleError) as e:
            O.gqa(q, k, v, nh, kvh, do_rotary=False)
        assert e.value.kind == "InvalidAttribute"
    with pytest.raises(O.OracleError):  # q and kv head_dim differ
        O.gqa(*_gqa_inputs(kv_hidden=8), 4, 2, do_rotary=False)
    with pytest.raises(O.OracleError):  # key/value shapes differ
        O.gqa(*_gqa_inputs(v_hidden=6), 4, 2, do_rotary=False)


def test_gqa_with_rope_rotates_present_key():
    qr = (np.arange(16, dtype=f32) * f32(0.1) + f32(0.05)).reshape(1, 1, 16)
    kr = (np.arange(8, dtype=f32) * f32(0.2) + f32(0.1)).reshape(1, 1, 8)
    vr = (np.arange(8, dtype=f32) * f32(0.3)).reshape(1, 1, 8)
    cos, sin = _taylor_tables(8, 2)
    _, pk, _ = O.gqa(qr, kr, vr, 4, 2, np.zeros((1, 2, 1, 4), f32), np.zeros((1, 2, 1, 4), f32),
                     cos, sin, do_rotary=True)
    assert np.abs(pk[0, 0, 1] - kr[0, 0, :4]).max() > 1e-4


def test_gqa_matches_f64_bruteforce_with_rope():
    import smallaios_amd as S
    rng = np.random.default_rng(9)
    b, sq, nh, kvh, d, past = 2, 3, 8, 2, 32, 20
    q = rng.standard_normal((b, sq, nh * d)).astype(f32)
    k = rng.standard_normal((b, sq, kvh * d)).astype(f32)
    v = rng.standard_normal((b, sq, kvh * d)).astype(f32)
    pk = rng.standard_normal((b, kvh, past, d)).astype(f32)
    pv = rng.standard_normal((b, kvh, past, d)).astype(f32)
    cos, sin = S.rope_tables(64, d, 10000.0)
    attn, prk, prv = O.gqa(q, k, v, nh, kvh, pk, pv, cos, sin, do_rotary=True)

    def rope64(x, pos):
        c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
        x0, x1 = x[: d // 2], x[d // 2:]
        return np.concatenate([c * x0 - s * x1, s * x0 + c * x1])

    scale = 1 / math.sqrt(d)
    for bi in range(b):
        for h in range(nh):
            kh = h // (nh // kvh)
            keys = [pk[bi, kh, t].astype(np.float64) for t in range(past)]
            keys += [rope64(k[bi, i, kh * d:(kh + 1) * d].astype(np.float64), past + i) for i in range(sq)]
            vals = [pv[bi, kh, t].astype(np.float64) for t in range(past)]
            vals += [v[bi, i, kh * d:(kh + 1) * d].astype(np.float64) for i in range(sq)]
            K, V = np.array(keys), np.array(vals)
            for i in range(sq):
                qq = rope64(q[bi, i, h * d:(h + 1) * d].astype(np.float64), past + i)
                s = K[: past + i + 1] @ qq * scale
                p = np.exp(s - s.max())
                want = (p / p.sum()) @ V[: past + i + 1]
                np.testing.assert_allclose(attn[bi, i, h * d:(h + 1) * d], want, atol=3e-5, rtol=1e-4)
            np.testing.assert_allclose(prk[bi, kh, past:], K[past:], atol=1e-5)


# ---------------------------------------------------- KV quantisation spec ---
def _int8_numpy(x):
    amax = np.abs(x).max(axis=-1, keepdims=True)
    s = np.where(amax > 0, amax / f32(127.0), f32(1.0)).astype(f32)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = np.rint(x / s)
    r = np.nan_to_num(r, nan=0.0, posinf=127, neginf=-128)
    return np.clip(r, -128, 127).astype(np.int8), s[..., 0]


def test_int8_quant_matches_numpy_and_invariants():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((300, 128)).astype(f32) * rng.uniform(1e-3, 1e3, (300, 1)).astype(f32)
    x[0] = 0.0
    x[1, :] = 0.5 * (np.arange(128) % 3 - 1)  # ties after scaling
    want_c, want_s = _int8_numpy(x)
    for i in range(x.shape[0]):
        c, s = O.quant_int8_row(x[i])
        assert s.view(np.uint32) == want_s[i].view(np.uint32)
        np.testing.assert_array_equal(c, want_c[i])
        assert np.abs(c.astype(np.int32)).max() <= 127
        if np.abs(x[i]).max() > 0:
            assert np.abs(c.astype(np.int32)).max() == 127
            assert np.abs(c.astype(f32) * s - x[i]).max() <= s * 0.5 * (1 + 1e-6)
    assert O.quant_int8_row(np.zeros(64, f32))[1] == 1.0


def _round_half_away(x):
    t = np.trunc(x)
    fr = x - t
    return np.where(fr >= 0.5, t + 1, np.where(fr <= -0.5, t - 1, t))


def _int4_numpy(x):
    g = x.reshape(-1, 32)
    mn, mx = g.min(axis=1), g.max(axis=1)
    rng_ = (mx - mn).astype(f32)
    sc = np.where(rng_ > 0, rng_ / f32(15.0), f32(1.0)).astype(f32)
    s16, z16 = sc.astype(np.float16), mn.astype(np.float16)
    sf, zf = s16.astype(f32), z16.astype(f32)
    q = _round_half_away((g - zf[:, None]) / sf[:, None])
    q = np.clip(q, 0, 15).astype(np.uint32)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    return packed, s16.view(np.uint16), z16.view(np.uint16), q.reshape(-1)


def test_int4_quant_matches_numpy_and_invariants():
    rng = np.random.default_rng(13)
    for trial in range(200):
        x = (rng.standard_t(3, 128) * rng.uniform(0.01, 50)).astype(f32)
        x[[7, 31, 64, 100]] *= 20
        if trial == 0:
            x[:32] = 1.25  # zero range group
        p, s, z = O.quant_int4_row(x)
        wp, ws, wz, q = _int4_numpy(x)
        np.testing.assert_array_equal(p, wp)
        np.testing.assert_array_equal(s, ws)
        np.testing.assert_array_equal(z, wz)
        deq = O.dequant_int4_row(p, s, z, 128)
        sf = s.view(np.float16).astype(f32).repeat(32)
        zf = z.view(np.float16).astype(f32).repeat(32)
        np.testing.assert_array_equal(deq, q.astype(f32) * sf + zf)
        # error bound: half a step plus the zero point's f16 rounding
        assert (np.abs(deq - x) <= 0.5 * sf + np.abs(zf) * 2 ** -10 + 1e-6 + sf * 1e-3).all()


def test_int4_zero_minimum_keeps_first_zero_sign():
    """The reference's scan (`if v < min { min = v }`, kv_compression.rs:227-235) keeps
    the first of equal minima, so a zero minimum is stored with the sign of the group's
    first zero: 0x8000 when -0 comes first, 0x0000 when +0 does. A min() that prefers
    either sign fails one of the two groups."""
    x = (np.abs(np.random.default_rng(5).standard_normal(64)) + 0.25).astype(f32)
    x[3], x[10] = f32(0.0), f32(-0.0)         # group 0: +0 first
    x[32 + 2], x[32 + 20] = f32(-0.0), f32(0.0)  # group 1: -0 first
    _, s, z = O.quant_int4_row(x)
    assert z.tolist() == [0x0000, 0x8000]
    # both groups keep their scale max / 15 and code zeros as 0
    p, _, _ = O.quant_int4_row(x)
    codes = np.stack([p & 15, p >> 4], axis=1).reshape(-1)
    assert codes[3] == codes[10] == codes[34] == codes[52] == 0
