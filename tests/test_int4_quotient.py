"""The int4 page append's quotient fast path, checked on the CPU.

kv_append_page_int4_kernel codes an element as med3(floor(fma(x - z, rcp(s), 1/2)), 0, 15)
where that value lies at least 2^-14 from every integer, and takes the reference's own
steps (the correctly rounded quotient, round_f32, `as u32`, min 15;
onnx-rt/src/kv_compression.rs:27-37 and :223-253) elsewhere. This emulates the fast path
in numpy: the fma with one rounding, v_rcp_f32 as the correctly rounded reciprocal moved by
-1, 0 or +1 ulp. It checks the fast path against round_f32 of the correctly rounded
quotient on random groups, with a third of the values placed on the half-integer ties
z + (k + 1/2) s, where a plausible mistake (floor without the half, a one-sided band, no
clamp) changes codes.
"""
import numpy as np

F32 = np.float32


def reference_codes(x, zf, sf):
    """round_f32((x - z) / s) as u32, min 15; the quotient correctly rounded."""
    d = (x - zf).astype(F32)
    t = (d.astype(np.float64) / sf.astype(np.float64)).astype(F32)
    with np.errstate(invalid="ignore"):
        tr = np.where(np.isnan(t), F32(0), np.trunc(np.clip(t, -2.1e9, 2.1e9))).astype(F32)
        fr = (t - tr).astype(F32)
        rr = np.where(fr >= 0.5, tr + 1, np.where(fr <= -0.5, tr - 1, tr)).astype(F32)
        v = np.where(np.isnan(rr) | (rr <= 0), 0.0, np.minimum(rr, 4e9))
    return np.minimum(v.astype(np.uint64), 15)


def fast_codes(x, zf, sf, rng):
    """The kernel's fast path; returns (codes, mask of elements it decides)."""
    d = (x - zf).astype(F32)
    r0 = (1.0 / sf.astype(np.float64)).astype(F32)
    up = np.nextafter(r0, F32(np.inf)).astype(F32)
    dn = np.nextafter(r0, F32(-np.inf)).astype(F32)
    pick = rng.integers(0, 3, len(r0))
    rf = np.where(pick == 0, r0, np.where(pick == 1, up, dn)).astype(F32)
    y = (d.astype(np.float64) * rf.astype(np.float64) + 0.5).astype(F32)  # fma: one rounding
    c = np.floor(y).astype(F32)
    fr = (y - c).astype(F32)
    with np.errstate(invalid="ignore"):
        decided = (fr >= F32(2.0 ** -14)) & (fr <= F32(1 - 2.0 ** -14))
    return np.clip(c, 0, 15).astype(np.uint64), decided


def test_int4_quotient_fast_path_matches_round_f32():
    rng = np.random.default_rng(0x1447)
    n = 250_000
    decided_total = 0
    for mag in (1e-3, 1.0, 30.0, 1e3):
        mn = (rng.standard_normal(n) * mag).astype(F32)
        width = (np.abs(rng.standard_normal(n)) * mag + 1e-5).astype(F32)
        sf = (width / F32(15)).astype(np.float16).astype(F32)
        zf = mn.astype(np.float16).astype(F32)
        x = (mn + rng.uniform(-0.02, 1.02, n).astype(F32) * width).astype(F32)
        k = rng.integers(0, 16, n)
        ties = rng.random(n) < 0.33
        x = np.where(ties, (zf + (k + F32(0.5)) * sf).astype(F32), x).astype(F32)
        keep = (sf > 0) & np.isfinite(sf) & np.isfinite(zf)
        x, zf, sf = x[keep], zf[keep], sf[keep]
        codes, decided = fast_codes(x, zf, sf, rng)
        ref = reference_codes(x, zf, sf)
        assert np.array_equal(codes[decided], ref[decided]), f"magnitude {mag}"
        # the band leaves only the elements near a tie to the slow path
        assert decided.mean() > 0.6
        decided_total += int(decided.sum())
    assert decided_total > 600_000
