"""head_dim 256 (the Gemma 3 attention shape, onnx-rt/src/model_loader/config.rs:695-717:
8 query heads over 4 kv heads, sliding windows of 1024) through kernels 1-3 on the
int8 and the int4 cache (every case runs for both), against the oracle. Same bar as
the other parity tests: codes and scales bit-exact, outputs within 2e-3 abs + 1e-2
rel. The int4 decode runs head_dim 256 as two 128-dim halves of its 128 layout; the
int4 prefill keeps one LDS tile (f16 hi + lo K and V, 109 KB) behind two barriers.
"""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import Case, assert_close, err_tol_ratio, log, outlier_keys

pytestmark = pytest.mark.gpu
D = 256


@pytest.fixture(params=[S.KV_INT8, S.KV_INT4], ids=["int8", "int4"])
def quant(request):
    return request.param


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    r = S.Runtime(0)
    yield r
    r.close()


@pytest.mark.parametrize("interleaved,kv_dtype", [(False, "bf16"), (True, "f32")])
def test_append_d256_bit_exact(rt, quant, interleaved, kv_dtype):
    log(f"append d=256 quant={quant} interleaved={interleaved} {kv_dtype}")
    c = Case(rt, 256 + interleaved, 3, 8, 4, D, [40, 5, 17], 9, theta=1e6, kv_dtype=kv_dtype,
             permute_pages=True, interleaved=interleaved, quant=quant)
    c.step_kv()
    c.check_codes()


@pytest.mark.parametrize("hq,hkv", [(8, 4), (4, 4), (4, 1)])
def test_decode_d256_groups(rt, quant, hq, hkv):
    log(f"decode d=256 quant={quant} hq={hq} hkv={hkv}")
    c = Case(rt, 300 + hq + hkv, 2, hq, hkv, D, [700, 129], 1, theta=1e6, permute_pages=True, quant=quant)
    c.step_kv()
    q = c.query("bf16")
    assert_close(c.gpu_decode(q, "bf16"), c.oracle_attend(q), f"d=256 group {hq // hkv}")
    c.check_codes(seqs=[1])


@pytest.mark.parametrize("split", [64, 1024])
def test_decode_d256_split_merge_and_fused(rt, quant, split):
    """Several split partials through the combine kernel, then the fused
    append + decode step."""
    log(f"decode d=256 split={split}")
    c = Case(rt, 333, 3, 8, 4, D, [2500, 1, 640], 1, theta=1e6, permute_pages=True,
             extra_tokens=1, quant=quant)
    prev = rt.set_decode_split(split)
    try:
        c.step_kv()
        q = c.query()
        assert_close(c.gpu_decode(q), c.oracle_attend(q), f"d=256 split {split}")
        c.cache.advance()
        q = c.query()
        got = c.step_fused(q)
        assert_close(got, c.oracle_attend(q), f"d=256 fused split {split}")
        c.check_codes(seqs=[1])
    finally:
        rt.set_decode_split(prev)


def test_decode_d256_windows(rt, quant):
    """Gemma 3's sliding layers: a layer window of 1024 and a mask window."""
    log("decode d=256 windows")
    c = Case(rt, 345, 2, 8, 4, D, [3000, 700], 1, theta=1e6, quant=quant)
    c.cache.set_layer_window(0, 1024)
    c.step_kv()
    q = c.query()
    assert_close(c.gpu_decode(q), c.oracle_attend(q, layer_window=1024), "d=256 layer window")
    assert_close(c.gpu_decode(q, window=300), c.oracle_attend(q, layer_window=1024, mask_window=300),
                 "d=256 both windows")


def test_decode_d256_group8(rt, quant):
    """Group 8 at head_dim 256: int8 decodes it (one wave per SIMD, the
    combine kernel over 2048 (head, dim) entries in two rounds of 1024
    threads), through one split, many splits merged in-kernel and by the
    combine kernel, and the fused step, with outlier keys; int4 rejects it
    as Unsupported."""
    log(f"decode d=256 group 8 quant={quant}")
    c = Case(rt, 346, 3, 16, 2, D, [64, 2100, 900], 1, quant=quant, theta=1e6,
             permute_pages=True, extra_tokens=1, k_transform=outlier_keys(D))
    c.step_kv()
    if quant == S.KV_INT4:
        with pytest.raises(S.SaiError) as e:
            c.gpu_decode(c.query())
        assert e.value.kind == "Unsupported"
        return
    q = c.query("bf16")
    ref = c.oracle_attend(q)
    # 512 and 1024: two or more tiles per wave, so the single tile buffer is
    # refilled with the next tile while the second pass of heads still needs
    # the current one's K codes
    for split, merge in ((0, 2), (256, 0), (256, 1), (512, 1), (1024, 0), (1024, 1)):
        prev_s, prev_m = rt.set_decode_split(split), rt.set_decode_merge(merge)
        try:
            got = c.gpu_decode(q, "bf16")
        finally:
            rt.set_decode_split(prev_s)
            rt.set_decode_merge(prev_m)
        log(f"  split {split} merge {merge}: worst err/tol {err_tol_ratio(got, ref):.4f}")
        assert_close(got, ref, f"d=256 group 8 split {split} merge {merge}")
    c.cache.advance()
    q = c.query("bf16")
    assert_close(c.step_fused(q, "bf16"), c.oracle_attend(q), "d=256 group 8 fused")
    c.check_codes(seqs=[1])


@pytest.mark.parametrize("hq,hkv,past,new,qd", [
    (8, 4, [300, 0], 150, "bf16"), (8, 1, [100, 37], 70, "f32"), (4, 4, [64, 640], 33, "f32")])
def test_prefill_d256(rt, quant, hq, hkv, past, new, qd):
    log(f"prefill d=256 hq={hq} hkv={hkv} past={past} new={new} {qd}")
    c = Case(rt, 350 + new, len(past), hq, hkv, D, past, new, theta=1e6, permute_pages=True,
             kv_dtype=qd, quant=quant)
    c.step_kv()
    c.check_codes()
    q = c.query(qd)
    assert_close(c.gpu_prefill(q, qd), c.oracle_attend(q), "d=256 prefill")


def test_prefill_d256_outlier_keys_and_window(rt, quant):
    """x20 outlier channels (Student-t elsewhere) and a 64-key sliding window."""
    log("prefill d=256 outlier keys + window")

    def outliers(rng, k):
        b, n, hd = k.shape
        t = rng.standard_t(3, size=k.shape).astype(np.float32).reshape(b, n, hd // D, D)
        t[..., [5, 17, 130, D - 3]] *= 20.0
        return t.reshape(b, n, hd)

    c = Case(rt, 360, 2, 8, 4, D, [200, 31], 90, theta=1e6, kv_dtype="bf16",
             k_transform=outliers, quant=quant)
    c.step_kv()
    q = c.query("bf16")
    assert_close(c.gpu_prefill(q, "bf16"), c.oracle_attend(q), "d=256 outlier prefill")
    assert_close(c.gpu_prefill(q, "bf16", window=64), c.oracle_attend(q, mask_window=64),
                 "d=256 windowed prefill")


@pytest.mark.parametrize("hq,hkv", [(8, 4), (16, 4)])
def test_decode_d256_outlier_keys(rt, quant, hq, hkv):
    """Student-t keys with x20 outlier channels at head_dim 256, fused step."""
    log(f"decode d=256 outlier K quant={quant} hq={hq} hkv={hkv}")
    c = Case(rt, 370 + hq, 3, hq, hkv, D, [3000, 700, 65], 1, theta=1e6, kv_dtype="bf16",
             permute_pages=True, k_transform=outlier_keys(D, (7, 63, 130, 200)),
             extra_tokens=1, quant=quant)
    c.step_kv()
    c.cache.advance()
    q = c.query("bf16")
    got = c.step_fused(q, "bf16")
    ref = c.oracle_attend(q)
    log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
    assert_close(got, ref, "d=256 outlier K")
    c.check_codes(seqs=[2])
