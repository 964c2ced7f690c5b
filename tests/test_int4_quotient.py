"""The int4 page append's shortcuts past IEEE division, checked on the CPU.

kv_append_page_int4_kernel takes two shortcuts, each with the reference's own steps
as the fallback (onnx-rt/src/kv_compression.rs:27-37 and :223-253):

* the group scale range / 15 as q0 = range * RN(1/15) corrected once by its fma residual,
  q0 + fma(-q0, 15, range) * RN(1/15); checked against the IEEE quotient for every
  positive finite f32 (a C program, OpenMP over the 2^31 inputs);
* the code of an element as med3(rint((x - z) * rcp(s)), 0, 15) where that product lies
  at least 2^-14 from every half-integer. Emulated in numpy (v_rcp_f32 as the correctly
  rounded reciprocal moved by -1, 0 or +1 ulp) and checked against round_f32 of the
  correctly rounded quotient on random groups, with a third of the values placed on the
  half-integer ties z + (k + 1/2) s, where a plausible mistake (floor instead of rint, a
  one-sided band, no clamp) changes codes.
"""
import os
import subprocess

import numpy as np
import pytest

F32 = np.float32

DIV_C = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
/* argv[1]: the divisor y; argv[2]: the kernel's constant RN(1/y) as a hex float */
int main(int argc, char** argv) {
  if (argc != 3) return 3;
  const float y = strtof(argv[1], NULL), c = strtof(argv[2], NULL);
  if (c != 1.0f / y) return 2;
  unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (long long b = 1; b < 0x7F800000LL; ++b) {
    const uint32_t u = (uint32_t)b;
    float r, want, q0, q;
    memcpy(&r, &u, 4);
    want = r / y;
    q0 = r * c;
    q = fmaf(fmaf(-q0, y, r), c, q0);
    if (memcmp(&q, &want, 4) != 0) ++bad;
  }
  printf("%llu\n", bad);
  return 0;
}
"""


@pytest.fixture(scope="module")
def div_exe(tmp_path_factory):
    d = tmp_path_factory.mktemp("div")
    src, exe = d / "div.c", d / "div"
    src.write_text(DIV_C)
    subprocess.run(["gcc", "-O2", "-fopenmp", "-o", str(exe), str(src), "-lm"], check=True)
    return exe


# (divisor, the kernels' constant): the int4 group scale range / 15, and the
# int8 page append's token scale amax / 127
@pytest.mark.parametrize("y,c", [("15", "0x1.111112p-4"), ("127", "0x1.020408p-7")])
def test_scale_division_exhaustive(div_exe, y, c):
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([str(div_exe), y, c], check=True, stdout=subprocess.PIPE, text=True,
                         env=env, timeout=600).stdout
    assert out.strip() == "0", f"{out.strip()} inputs where the corrected product differs"


def test_scale_division_needs_the_correction():
    """The plain product range * RN(1/15) is not the IEEE quotient everywhere, so the
    exhaustive check above is what pins the corrected form."""
    rng = np.random.default_rng(15)
    r = rng.uniform(1e-3, 1e3, 200_000).astype(F32)
    want = (r.astype(np.float64) / 15.0).astype(F32)
    plain = (r * F32(1.0 / 15.0)).astype(F32)
    assert np.any(plain != want)


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
    t = (d * rf).astype(F32)
    r = np.rint(t).astype(F32)  # round half to even, as v_rndne_f32
    with np.errstate(invalid="ignore"):
        decided = np.abs((t - r).astype(F32)) <= F32(0.5 - 2.0 ** -14)
    return np.clip(r, 0, 15).astype(np.uint64), decided


@pytest.mark.parametrize("mag", [1e-3, 1.0, 30.0, 1e3])
def test_int4_quotient_fast_path_matches_round_f32(mag):
    rng = np.random.default_rng(0x1447 + int(mag * 1000))
    n = 250_000
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
    # and the ties themselves go there
    assert decided[ties[keep]].mean() < 0.05
