"""Pins of the oracle's TurboQuant restatement (oracle/sai_oracle.c, TurboQuant
section; onnx-rt/src/kv_compression.rs).

Restated reference tests (kv_compression.rs:1021-1310): wht_known_vector,
wht_known_vector_alternating, wht_self_inverse_roundtrip,
encode_decode_roundtrip_{4,3,8}bit, reject_{non_power_of_two,zero}_dim,
reject_invalid_bits, deterministic_same_seed, different_seeds_different_signs,
constant_input_roundtrip, qjl_sign_captures_correct_signs,
qjl_correction_nonneg_identical, qjl_correction_improves_inner_product,
qjl_empty_vectors, qjl_zero_residual, cache_write_read_roundtrip.

Closed forms beside them: the butterfly on a one-hot vector gives the
Sylvester Hadamard column (-1)^popcount(i & j) / sqrt(n), which fixes the
pairing order; the rotation preserves norms and inner products; a code
decodes to within half a step of the rotated value (the quantiser's bound,
which a wrong rounding or scale breaks); the popcount correction equals
C_a C_b <s_a, s_b> / D computed from +-1 vectors; the sign vector is
balanced and seed-specific; the cache seeds follow the reference's mixing
constant. The attention estimator (sai_or_tq_attend) and the design's two
primitives (sai_or_tq_attention_logits, sai_or_tq_weighted_value_sum) are
checked against numpy evaluations built from the pinned pieces, and the
attention against softmax(scale * logits) then the weighted sum.
"""
import numpy as np
import pytest

import oracle as O


def test_reference_wht_kats():
    assert np.allclose(O.wht([1, 1, 1, 1], [1] * 4), [2, 0, 0, 0], atol=1e-6)
    assert np.allclose(O.wht([1, -1, 1, -1], [1] * 4), [0, 2, 0, 0], atol=1e-6)
    sg = [1, -1, 1, 1, -1, -1, 1, -1]
    x = np.arange(1, 9, dtype=np.float32)
    back = O.wht(O.wht(x, sg), sg, inverse=True)
    assert np.abs(back - x).max() < 1e-4


@pytest.mark.parametrize("n", [4, 16, 64, 128, 256])
def test_wht_is_the_sylvester_hadamard(n):
    norm = O.wht(np.eye(n, dtype=np.float32)[1], [1] * n)[0] * 1.0  # scale of one entry
    s = 1.0 / np.sqrt(n)
    assert abs(abs(norm) - s) < 1e-6
    for j in (0, 1, n // 2 - 1, n - 1):
        col = O.wht(np.eye(n, dtype=np.float32)[j], [1] * n)
        want = np.array([(-1) ** bin(i & j).count("1") for i in range(n)]) * s
        assert np.abs(col - want).max() < 1e-6, j


def test_rotation_preserves_norms_and_products():
    rng = np.random.default_rng(0)
    sg = O.tq_signs(7, 128)
    a, b = rng.standard_normal((2, 128)).astype(np.float32)
    ra, rb = O.wht(a, sg), O.wht(b, sg)
    assert abs(np.dot(ra, rb) - np.dot(a, b)) < 1e-3
    assert abs(np.linalg.norm(ra) - np.linalg.norm(a)) < 1e-4


@pytest.mark.parametrize("dim,bits,seed,slope,offset,slack", [
    (64, 4, 42, 0.1, -3.0, 0.1), (32, 3, 123, 0.2, -2.0, 0.2), (16, 8, 999, 0.5, -4.0, None)])
def test_reference_roundtrip_bounds(dim, bits, seed, slope, offset, slack):
    sg = O.tq_signs(seed, dim)
    x = (np.arange(dim, dtype=np.float32) * np.float32(slope) + np.float32(offset)).astype(np.float32)
    packed, sc, z, mn, mx = O.tq_encode(x, bits, sg)
    dec = O.tq_decode(packed, dim, bits, sc, z, sg)
    err = np.abs(dec - x).max()
    if slack is None:
        assert err < 0.5
    else:
        assert err < (mx - mn) / ((1 << bits) - 1) + slack
    # the quantiser's own bound in the rotated domain: half a step
    rot = O.wht(x, sg)
    codes = O.unpack_bits(packed, dim, bits).astype(np.float32)
    assert np.abs(codes * np.float32(sc) + np.float32(z) - rot).max() <= sc / 2 + 1e-5
    assert z == mn and np.isclose(sc, (mx - mn) / ((1 << bits) - 1))


def test_reference_rejections_and_determinism():
    x = np.zeros(17, np.float32)
    with pytest.raises(O.OracleError):
        O.tq_encode(x, 4, np.ones(17, np.int8))
    with pytest.raises(O.OracleError):
        O.tq_encode(np.zeros(16, np.float32), 5, np.ones(16, np.int8))
    a, b = O.tq_signs(42, 64), O.tq_signs(42, 64)
    assert np.array_equal(a, b)
    assert not np.array_equal(O.tq_signs(42, 64), O.tq_signs(99, 64))
    inp = np.arange(64, dtype=np.float32) * np.float32(0.1)
    e1, e2 = O.tq_encode(inp, 4, a), O.tq_encode(inp, 4, b)
    assert np.array_equal(e1[0], e2[0]) and e1[1:3] == e2[1:3]
    s = O.tq_signs(1234, 4096)
    assert set(np.unique(s)) == {-1, 1} and abs(int(s.sum())) < 300
    assert np.array_equal(O.tq_signs(0, 32), O.tq_signs(0x5EEDDEADBEEFCAFE, 32))


def test_reference_constant_input():
    sg = O.tq_signs(42, 16)
    x = np.full(16, 3.14, np.float32)
    p, sc, z, _, _ = O.tq_encode(x, 4, sg)
    assert np.abs(O.tq_decode(p, 16, 4, sc, z, sg) - x).max() < 1.5


def test_reference_qjl_kats():
    bits, c = O.qjl_encode([1.0, -2.0, 3.0, -4.0, 0.5, -0.5, 0.0, 1.0], np.zeros(8))
    assert int(bits[0]) & 0xFF == 0xD5
    assert c == pytest.approx((1 + 2 + 3 + 4 + 0.5 + 0.5 + 0 + 1) / 8)
    r, rc = O.qjl_encode([1.0, 2.0, 3.0, 4.0], [0.5, 1.5, 2.5, 3.5])
    assert O.qjl_correction(r, rc, r, rc, 4) >= 0.0
    assert O.qjl_correction(r, rc, r, rc, 4) == pytest.approx(rc * rc)
    z, zc = O.qjl_encode([1.0, 2.0, 3.0, 4.0], [1.0, 2.0, 3.0, 4.0])
    assert zc == 0.0
    assert O.qjl_correction(z, 0.0, z, 0.0, 0) == 0.0


def test_correction_matches_sign_vectors():
    rng = np.random.default_rng(3)
    for d in (16, 64, 100, 128):
        ra, rb = rng.standard_normal((2, d)).astype(np.float32)
        ba, ca = O.qjl_encode(ra, np.zeros(d))
        bb, cb = O.qjl_encode(rb, np.zeros(d))
        sa, sb = np.where(ra >= 0, 1.0, -1.0), np.where(rb >= 0, 1.0, -1.0)
        want = ca * cb * float(sa @ sb) / d
        assert O.qjl_correction(ba, ca, bb, cb, d) == pytest.approx(want, rel=1e-6, abs=1e-7)


def test_reference_qjl_improves_inner_product():
    dim = 64
    sg = O.tq_signs(42, dim)
    a = (np.arange(dim, dtype=np.float32) * np.float32(0.1) - np.float32(3.0)).astype(np.float32)
    b = (np.arange(dim, dtype=np.float32) * np.float32(0.05) + np.float32(1.0)).astype(np.float32)
    true_dot = float(a @ b)
    da = O.tq_decode(*O.tq_encode(a, 4, sg)[:1], dim, 4, *O.tq_encode(a, 4, sg)[1:3], sg)
    db = O.tq_decode(*O.tq_encode(b, 4, sg)[:1], dim, 4, *O.tq_encode(b, 4, sg)[1:3], sg)
    quant_dot = float(da @ db)
    corr = O.qjl_correction(*O.qjl_encode(a, da), *O.qjl_encode(b, db), dim)
    assert abs(quant_dot + corr - true_dot) < abs(quant_dot - true_dot) * 2 + 1.0


def test_cache_seeds_and_write_rows():
    # CompressedKVCache::new: head_seed = seed * 0x9E3779B97F4A7C15 + (layer*nh + head)
    seed = 0xDEADBEEFCAFE1234
    want = (seed * 0x9E3779B97F4A7C15 + (2 * 8 + 3)) & (2**64 - 1)
    assert O.tq_head_seed(seed, 2, 8, 3) == want
    # cache_write_read_roundtrip (kv_compression.rs:1490-1514): error < 1
    rng = np.random.default_rng(5)
    sg = O.tq_signs(O.tq_head_seed(seed, 0, 1, 0), 64)
    x = (rng.standard_normal((10, 64)) * 0.5).astype(np.float32)
    codes, sc, z, sb, c = O.tq_write_rows(x, 4, sg, True)
    for t in range(10):
        dec = O.tq_decode(codes[t], 64, 4, sc[t], z[t], sg)
        assert np.abs(dec - x[t]).max() < 1.0
        bits, ct = O.qjl_encode(x[t], dec)
        assert np.array_equal(sb[t], bits) and ct == c[t]


@pytest.mark.parametrize("bits,qjl", [(4, True), (3, False), (8, True)])
def test_attend_matches_numpy_of_the_pinned_pieces(bits, qjl):
    rng = np.random.default_rng(bits)
    d, g, n = 64, 4, 37
    sg = O.tq_signs(77, d)
    k = rng.standard_normal((n, d)).astype(np.float32)
    v = rng.standard_normal((n, d)).astype(np.float32)
    q = rng.standard_normal((g, d)).astype(np.float32)
    ek, ev = O.tq_write_rows(k, bits, sg, qjl), O.tq_write_rows(v, bits, sg, qjl)
    got = O.tq_attend(q, bits, qjl, sg, ek, ev, 0.125)
    kd = np.stack([O.tq_decode(ek[0][t], d, bits, ek[1][t], ek[2][t], sg) for t in range(n)])
    vd = np.stack([O.tq_decode(ev[0][t], d, bits, ev[1][t], ev[2][t], sg) for t in range(n)])
    eq = O.tq_write_rows(q, bits, sg, qjl)
    for h in range(g):
        qd = O.tq_decode(eq[0][h], d, bits, eq[1][h], eq[2][h], sg).astype(np.float64)
        lg = kd.astype(np.float64) @ qd
        if qjl:
            lg += np.array([O.qjl_correction(eq[3][h], eq[4][h], ek[3][t], ek[4][t], d)
                            for t in range(n)])
        w = np.exp(0.125 * lg - (0.125 * lg).max())
        want = (w / w.sum()) @ vd
        np.testing.assert_allclose(got[h], want, atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("bits,qjl", [(4, True), (3, True), (8, False)])
def test_logits_and_weighted_sum(bits, qjl):
    rng = np.random.default_rng(10 + bits)
    d, g, n = 64, 2, 29
    sg = O.tq_signs(5, d)
    k = rng.standard_normal((n, d)).astype(np.float32)
    v = rng.standard_normal((n, d)).astype(np.float32)
    q = rng.standard_normal((g, d)).astype(np.float32)
    ek, ev = O.tq_write_rows(k, bits, sg, qjl), O.tq_write_rows(v, bits, sg, qjl)
    lg = O.tq_attention_logits(q, bits, qjl, sg, ek)
    eq = O.tq_write_rows(q, bits, sg, qjl)
    kd = np.stack([O.tq_decode(ek[0][t], d, bits, ek[1][t], ek[2][t], sg) for t in range(n)])
    vd = np.stack([O.tq_decode(ev[0][t], d, bits, ev[1][t], ev[2][t], sg) for t in range(n)])
    for h in range(g):
        qd = O.tq_decode(eq[0][h], d, bits, eq[1][h], eq[2][h], sg).astype(np.float64)
        want = kd.astype(np.float64) @ qd
        if qjl:
            want += [O.qjl_correction(eq[3][h], eq[4][h], ek[3][t], ek[4][t], d) for t in range(n)]
        np.testing.assert_allclose(lg[h], want, atol=1e-4, rtol=1e-5)
    w = rng.random((g, n)).astype(np.float32)
    ws = O.tq_weighted_value_sum(w, bits, sg, ev)
    np.testing.assert_allclose(ws, w.astype(np.float64) @ vd, atol=1e-4, rtol=1e-5)
    # attention = weighted sum of softmax(scale * logits)
    sc = 0.125
    p = np.exp(sc * (lg - lg.max(1, keepdims=True)))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(O.tq_attend(q, bits, qjl, sg, ek, ev, sc),
                               O.tq_weighted_value_sum(p, bits, sg, ev), atol=2e-5, rtol=1e-4)
