"""Prefill of short chunks over long pasts, where the host cuts the rows' key
range into splits (fewer than 256 workgroups, at least 16 tiles to stream):
each workgroup streams its split's tiles and writes (m, l, o) partials, and the
decode's combine kernel merges them, every row of the chunk as a sequence of
its own. Against the oracle at the prefill bar (2e-3 abs + 1e-2 rel; bf16
outputs with bf16's rounding on top; large V against the weighted bound of
the precise pass), for int8 and int4, head_dim 64/128/168/256, groups 1-8,
windows, and ragged pasts (rows whose visible range ends before a split
starts write empty partials). Chunks large enough for the plain grid are the
other prefill tests' (the c5 chunk among them).
"""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import (Case, assert_close, assert_close_weighted, bf16_tol_close,
                       err_tol_ratio, log, outlier_keys, weighted_abs_v)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    assert S.lib().sai_device_supported(0) == 1, "device 0 is not gfx950"
    r = S.Runtime(0)
    yield r
    r.close()


CASES = [
    # quant, hq, hkv, d, past, new, window, out dtype, outlier keys
    (S.KV_INT8, 32, 8, 128, [8000], 16, 0, "f32", False),
    (S.KV_INT8, 8, 1, 64, [9000], 1, 0, "f32", False),
    (S.KV_INT4, 32, 8, 128, [5000, 3000], 4, 0, "bf16", True),
    (S.KV_INT8, 16, 2, 256, [6000], 33, 700, "f32", True),
    (S.KV_INT8, 32, 8, 168, [4000, 10], 64, 0, "f32", False),
    (S.KV_INT4, 8, 4, 256, [3000, 100], 20, 0, "f32", False),
    (S.KV_INT8, 16, 4, 128, [2500, 0, 1200], 90, 300, "bf16", False),
    (S.KV_INT4, 16, 2, 64, [7000], 8, 0, "f32", True),
]


@pytest.mark.parametrize("case", CASES, ids=[f"case{i}" for i in range(len(CASES))])
def test_prefill_key_split(rt, case):
    quant, hq, hkv, d, past, new, window, od, outl = case
    log(f"prefill key split: quant {quant} hq {hq} hkv {hkv} d {d} past {past} new {new} "
        f"window {window} out {od} outlier keys {outl}")
    c = Case(rt, 0x4B5 + d + new, len(past), hq, hkv, d, past, new, theta=5e5, quant=quant,
             permute_pages=True, kv_dtype="bf16",
             k_transform=outlier_keys(d, (7, 31, 50, 60)) if outl else None)
    c.step_kv()
    q = c.query("bf16")
    got = c.gpu_prefill(q, "bf16", window=window, out_dtype=od)
    ref = c.oracle_attend(q, mask_window=window)
    if od == "bf16":
        bf16_tol_close(got, ref, "prefill key split (bf16 out)")
    else:
        log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
        assert_close(got, ref, "prefill key split")


@pytest.mark.parametrize("quant,vscale", [(S.KV_INT8, 1.0e5), (S.KV_INT4, 1.0e4)])
def test_prefill_key_split_large_v(rt, quant, vscale):
    """Large V with the key split: int8 splits whose tiles hold large V scales
    run the precise pass and store their partials in true units (its
    accumulator is in units of 2^(vexp - 12)); the merge then weighs them
    against the fast splits'."""
    log(f"prefill key split, V x{vscale:g}, quant {quant}")
    c = Case(rt, 0x4B6, 1, 16, 4, 128, [5000], 24, theta=5e5, quant=quant,
             v_transform=lambda rng, v: v * np.float32(vscale))
    c.step_kv()
    q = c.query("f32")
    got = c.gpu_prefill(q, "f32")
    ref = c.oracle_attend(q)
    assert np.isfinite(got).all()
    kappa = 2.0 ** -12 if quant == S.KV_INT8 else 2.0 ** -9
    r = assert_close_weighted(got, ref, weighted_abs_v(c, q), kappa, "prefill key split, large V")
    log(f"  worst err / weighted bound {r:.4f}")


def test_prefill_key_split_repeated_and_reused(rt):
    """The same short chunk twice (the precise pass's flags and the partials
    are reused): bit-identical results, equal to the oracle's."""
    log("prefill key split: repeated")
    c = Case(rt, 0x4B7, 2, 32, 8, 128, [6000, 2000], 12, theta=5e5, permute_pages=True)
    c.step_kv()
    q = c.query("f32")
    a = c.gpu_prefill(q, "f32")
    b = c.gpu_prefill(q, "f32")
    assert np.array_equal(a, b)
    assert_close(a, c.oracle_attend(q), "prefill key split, first")
