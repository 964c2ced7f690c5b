"""Pins of the oracle's RoPE-table restatement (oracle/sai_oracle.c,
precompute_rope_tables of onnx-rt/src/model_loader/gemma.rs:458-541).

The reference holds one test of these tables, precompute_rope_tables_has_expected_size
(gemma.rs:769-783: 16 x 4 entries, row 0 = (1, 0) within 1e-2); it is restated
below. The rest is pinned by what the mathematics fixes, with tolerances taken
from each approximation's truncation remainder, so that a dropped series term,
a wrong constant or a transposed index fails:

* ln_approx: atanh series to y^7, remainder <= 2 y^9 / (9 (1 - y^2)) <= 1.3e-5
  for y <= 1/3; dropping the y^7 term costs 1.3e-4 near mantissa 2.
* exp_approx: Taylor to r^5 on r in [0, ln 2), relative remainder
  <= r^6 / 720 <= 1.6e-4; dropping r^5/120 costs up to 1.4e-3.
* sin_approx / cos_approx: Taylor to y^9 on [-pi, pi], remainder
  <= pi^11 / 11! = 7.4e-3; dropping y^9 costs up to 0.082.
* exp_approx(0) == 1 exactly, so column 0 of every table holds bf16 of the
  approximations at angle = pos, which must sit within the sin bound plus half
  a bf16 ulp of cos(pos), sin(pos); at small positions every column sits near
  cos/sin(pos * theta^(-2i/d)), which pins the exponent 2i/d.

The standalone RotaryEmbedding rotation itself is the oracle's apply_rope,
pinned in test_oracle.py by the reference's own KATs.
"""
import numpy as np
import pytest

import oracle as O

L = O.lib()


def test_floor_approx_known_values():
    cases = {2.5: 2.0, -2.5: -3.0, 3.0: 3.0, -3.0: -3.0, 0.0: 0.0, 1e-8: 0.0, -1e-8: -1.0,
             1303.7: 1303.0, -0.5: -1.0}
    for x, want in cases.items():
        assert L.sai_or_floor_approx(x) == want, x


def test_ln_approx_within_series_remainder():
    xs = np.concatenate([np.logspace(-3, 7, 4001), [2.0 ** k * 1.999 for k in range(-8, 22)],
                         [1.0, 2.0, 10000.0, 500000.0, 1e6]]).astype(np.float32)
    got = np.array([L.sai_or_ln_approx(float(x)) for x in xs], np.float64)
    err = np.abs(got - np.log(xs.astype(np.float64)))
    assert err.max() < 3e-5, (xs[err.argmax()], err.max())
    # the y^7 term is needed: its size near mantissa 2 is above the tolerance
    y = (1.999 - 1) / (1.999 + 1)
    assert 2 * y ** 7 / 7 > 1e-4
    assert L.sai_or_ln_approx(0.0) == -np.inf and L.sai_or_ln_approx(-1.0) == -np.inf


def test_exp_approx_within_taylor_remainder():
    xs = np.linspace(-20.0, 20.0, 8001).astype(np.float32)
    got = np.array([L.sai_or_exp_approx(float(x)) for x in xs], np.float64)
    rel = np.abs(got / np.exp(xs.astype(np.float64)) - 1.0)
    assert rel.max() < 2e-4, (xs[rel.argmax()], rel.max())
    assert L.sai_or_exp_approx(0.0) == 1.0
    assert np.log(2.0) ** 5 / 120 > 1e-3  # a dropped r^5 term would show


def test_sin_cos_approx_within_taylor_remainder():
    xs = np.linspace(-100.0, 100.0, 20001).astype(np.float32)
    s = np.array([L.sai_or_sin_approx(float(x)) for x in xs], np.float64)
    c = np.array([L.sai_or_cos_approx(float(x)) for x in xs], np.float64)
    x64 = xs.astype(np.float64)
    bound = np.pi ** 11 / 39916800 + 1e-4
    assert np.abs(s - np.sin(x64)).max() < bound
    assert np.abs(c - np.cos(x64)).max() < bound
    assert L.sai_or_sin_approx(0.0) == 0.0


def test_reference_kat_expected_size_and_row0():
    # gemma.rs:769-783
    c, s = O.rope_tables_bf16(16, 4, 10_000.0)
    assert c.nbytes == 16 * 4 * 2 and s.nbytes == 16 * 4 * 2
    cf, sf = O.bf16_bits_to_f32(c[0]), O.bf16_bits_to_f32(s[0])
    assert np.all(np.abs(cf - 1.0) < 1e-2) and np.all(np.abs(sf) < 1e-2)
    assert np.all(sf == 0.0)  # sin_approx(0) is exactly 0


@pytest.mark.parametrize("theta,half", [(10_000.0, 64), (1_000_000.0, 128), (500_000.0, 32)])
def test_tables_against_closed_forms(theta, half):
    max_pos = 512
    c, s = O.rope_tables_bf16(max_pos, half, theta)
    cf, sf = O.bf16_bits_to_f32(c).astype(np.float64), O.bf16_bits_to_f32(s).astype(np.float64)
    pos = np.arange(max_pos, dtype=np.float64)
    bf16_half_ulp = 2.0 ** -9
    sin_bound = np.pi ** 11 / 39916800
    # column 0: angle = pos exactly (exp_approx(0) == 1); reduction error grows with pos
    tol0 = sin_bound + bf16_half_ulp + 1e-4
    assert np.abs(cf[:, 0] - np.cos(pos)).max() < tol0
    assert np.abs(sf[:, 0] - np.sin(pos)).max() < tol0
    # every column at small positions: inv_freq = theta^(-2i/d) within 3e-4 relative
    d = 2 * half
    inv = theta ** (-(2.0 * np.arange(half)) / d)
    ang = pos[:17, None] * inv[None, :]
    tol = sin_bound + bf16_half_ulp + 16 * 3e-4
    assert np.abs(cf[:17] - np.cos(ang)).max() < tol
    assert np.abs(sf[:17] - np.sin(ang)).max() < tol
    # the tables are deterministic functions of (max_pos, half, theta): a
    # shorter table is a prefix of a longer one
    c2, s2 = O.rope_tables_bf16(64, half, theta)
    assert np.array_equal(c2, c[:64]) and np.array_equal(s2, s[:64])


def test_f32_to_bf16_bits_matches_scalar_oracle():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 10,
                        np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1.00390625,
                                  1.01171875], np.float32)])
    want = np.array([L.sai_or_f32_to_bf16(float(v)) for v in x], np.uint16)
    assert np.array_equal(O.f32_to_bf16_bits(x), want)
