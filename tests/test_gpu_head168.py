"""head_dim 168 (the Gemma 4 31B attention shape, onnx-rt/src/model_loader/config.rs:720-737:
32 query heads over 8 kv heads, sliding windows of 4096) through kernels 1-3 on the int8
cache, against the oracle.

The cache stores a 168-dim row as 192 dims: each 84-dim half of the split-half RoPE
pairing is followed by 12 zero dims. The kernels run at the stored width and read and
write the caller's 168-dim rows; sai_kvcache_read hands back the 168 codes of a row.
Same bar as the other parity tests: codes and scales bit-exact (the padding cannot move
a row's absolute maximum), outputs within 2e-3 abs + 1e-2 rel. int4 (groups of 32)
does not divide 168 and is rejected as Unsupported.
"""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import (Case, assert_close, assert_close_weighted, err_tol_ratio, log,
                       outlier_keys, weighted_abs_v)

pytestmark = pytest.mark.gpu
D = 168
THETA = 1e6


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    r = S.Runtime(0)
    yield r
    r.close()


# ----------------------------------------------------------------- append ---
@pytest.mark.parametrize("interleaved,rot,kv_dtype", [
    (False, True, "bf16"), (True, True, "f32"), (False, False, "f32"), (False, True, "f32")])
def test_append_d168_bit_exact(rt, interleaved, rot, kv_dtype):
    """The page-block kernel (the past, and 9 new tokens from starts 40, 5 and
    17: partial first and last pages), then 3 tokens and 1 token through the
    per-row kernel, all into one cache; K with x20 outlier channels in both
    halves, including the last dim of each."""
    log(f"append d=168 interleaved={interleaved} rotary={rot} {kv_dtype}")
    c = Case(rt, 0x168A + 2 * interleaved + rot, 3, 32, 8, D, [40, 5, 17], 9, theta=THETA,
             kv_dtype=kv_dtype, permute_pages=True, interleaved=interleaved, do_rotary=rot,
             extra_tokens=4, k_transform=outlier_keys(D, channels=(3, 83, 84, 130, 167)))
    c.step_kv()
    c.check_codes()
    c.cache.advance()
    k, v = c.kv(3)
    c.append_both(k, v)
    c.check_codes()
    c.cache.advance()
    k, v = c.kv(1)
    c.append_both(k, v)
    c.check_codes()


def test_append_d168_special_values(rt):
    """Zero rows, huge/tiny magnitudes, inf and NaN (in the first and the
    second half) keep the codes bit-exact; the 8 tokens take the page-block
    kernel."""
    log("append d=168 special values")

    def poison(rng, k):
        k = k.copy()
        k[0, 0, :D] = 0.0
        k[0, 1, :D] = np.float32(3.0e38)
        k[0, 2, :D] *= np.float32(1e-30)
        k[0, 3, 83] = np.inf
        k[0, 4, 84] = np.nan
        k[0, 5, :D] = np.nan
        k[0, 6, 100:D] = np.float32(-np.inf)
        return k

    c = Case(rt, 0x168B, 1, 4, 2, D, [0], 8, k_transform=poison, do_rotary=False)
    c.step_kv()
    c.check_codes()


# ----------------------------------------------------------------- decode ---
@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (16, 8), (64, 8)])
def test_decode_d168_groups(rt, hq, hkv):
    """Groups 4 (Gemma 4 31B), 1, 2 and 8; bf16 Q and K/V, ragged lengths."""
    log(f"decode d=168 hq={hq} hkv={hkv}")
    c = Case(rt, 0x168C + hq, 3, hq, hkv, D, [700, 129, 2000], 1, theta=THETA,
             kv_dtype="bf16", permute_pages=True)
    c.step_kv()
    q = c.query("bf16")
    got = c.gpu_decode(q, "bf16")
    ref = c.oracle_attend(q)
    log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
    assert_close(got, ref, f"d=168 group {hq // hkv}")
    c.check_codes(seqs=[1])


@pytest.mark.parametrize("split,merge", [(64, 0), (64, 1), (1024, 2)])
def test_decode_d168_split_merge_and_fused(rt, split, merge):
    """Split partials merged by the combine kernel and in-kernel, then the
    fused append + decode step (its appender wave writes the 168-dim row)."""
    log(f"decode d=168 split={split} merge={merge}")
    c = Case(rt, 0x168D + split, 3, 32, 8, D, [2500, 1, 640], 1, theta=THETA,
             permute_pages=True, extra_tokens=1)
    prev_s, prev_m = rt.set_decode_split(split), rt.set_decode_merge(merge)
    try:
        c.step_kv()
        q = c.query()
        assert_close(c.gpu_decode(q), c.oracle_attend(q), f"d=168 split {split}")
        c.cache.advance()
        q = c.query("bf16")
        got = c.step_fused(q, "bf16")
        assert_close(got, c.oracle_attend(q), f"d=168 fused split {split}")
        c.check_codes(seqs=[0, 1])
    finally:
        rt.set_decode_split(prev_s)
        rt.set_decode_merge(prev_m)


def test_decode_d168_windows_interleaved(rt):
    """Gemma 4's sliding layers (a layer window of 4096 over 6000 keys) and a
    mask window, with interleaved RoPE pairs."""
    log("decode d=168 windows, interleaved")
    c = Case(rt, 0x168E, 2, 32, 8, D, [6000, 900], 1, theta=THETA, interleaved=True)
    c.cache.set_layer_window(0, 4096)
    c.step_kv()
    q = c.query()
    assert_close(c.gpu_decode(q), c.oracle_attend(q, layer_window=4096), "d=168 layer window")
    assert_close(c.gpu_decode(q, window=300),
                 c.oracle_attend(q, layer_window=4096, mask_window=300), "d=168 both windows")


@pytest.mark.parametrize("split,merge", [(512, 0), (1024, 1), (2048, 1)])
def test_decode_d168_group8_long_splits(rt, split, merge):
    """Group 8 (two passes of four heads) with two or more tiles per wave: the
    single tile buffer is refilled with the next tile only after the second
    pass's QK has read the current one's K codes."""
    log(f"decode d=168 group 8 split={split} merge={merge}")
    c = Case(rt, 0x1690 + split, 3, 64, 8, D, [3000, 700, 65], 1, theta=THETA,
             permute_pages=True, k_transform=outlier_keys(D, (7, 63, 90, 150)))
    prev_s, prev_m = rt.set_decode_split(split), rt.set_decode_merge(merge)
    try:
        c.step_kv()
        q = c.query("bf16")
        got = c.gpu_decode(q, "bf16")
        ref = c.oracle_attend(q)
        log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
        assert_close(got, ref, f"d=168 group 8 split {split}")
    finally:
        rt.set_decode_split(prev_s)
        rt.set_decode_merge(prev_m)


@pytest.mark.parametrize("hq", [32, 64])
def test_decode_d168_outlier_keys(rt, hq):
    """Student-t keys with x20 outlier channels, fused step."""
    log(f"decode d=168 outlier K hq={hq}")
    c = Case(rt, 0x168F + hq, 3, hq, 8, D, [3000, 700, 65], 1, theta=THETA, kv_dtype="bf16",
             permute_pages=True, k_transform=outlier_keys(D, (7, 63, 90, 150)), extra_tokens=1)
    c.step_kv()
    c.cache.advance()
    q = c.query("bf16")
    got = c.step_fused(q, "bf16")
    ref = c.oracle_attend(q)
    log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
    assert_close(got, ref, "d=168 outlier K")
    c.check_codes(seqs=[2])


def test_decode_d168_bf16_output(rt):
    """bf16 attention output of the fused step (the reference's GPU GQA
    returns Q's dtype)."""
    from _gpu_util import bf16_tol_close
    log("decode d=168 bf16 output")
    c = Case(rt, 0x1690, 4, 32, 8, D, [4095, 1000, 17, 3000], 1, theta=THETA,
             kv_dtype="bf16", extra_tokens=1)
    q = c.query("bf16")
    got = c.step_fused(q, "bf16", out_dtype="bf16")
    r = bf16_tol_close(got, c.oracle_attend(q), "d=168 bf16 output")
    log(f"  worst err/tol {r:.4f}")


def test_decode_d168_large_v(rt):
    """|v| ~ 4e5 with keys at 300-339 scaled x6 (weights on a few keys whose
    V rows cancel), checked against the two-term int8 P' bound as at 128."""
    from _gpu_util import assert_close_decode_bound, decode_weight_bounds
    log("decode d=168 large V")

    def jump(rng, k):
        if k.shape[1] >= 340:
            k[:, 300:340] *= 6.0
        return k

    c = Case(rt, 0x1691, 3, 32, 8, D, [700, 450, 3000], 1, theta=THETA, kv_dtype="bf16",
             permute_pages=True, k_transform=jump, v_transform=lambda rng, v: v * np.float32(1e5))
    q = c.query("bf16")
    got = c.step_fused(q, "bf16")
    c.check_codes(seqs=[1])
    ref = c.oracle_attend(q)
    assert np.isfinite(got).all()
    wabs, rep = decode_weight_bounds(c, q)
    r = assert_close_decode_bound(got, ref, wabs, rep, "d=168 decode, large V")
    log(f"  worst err / bound {r:.4f}")


def test_decode_d168_layer_full_size(rt):
    """A Gemma 4 31B layer's decode at 8 x 8192 (32Q/8KV, bf16 Q and K/V):
    every output against the oracle, codes of two sequences."""
    log("decode d=168 layer: 8 x 8192, 32Q/8KV")
    c = Case(rt, 0x1692, 8, 32, 8, D, [8191] * 8, 1, theta=THETA, kv_dtype="bf16")
    q = c.query("bf16")
    got = c.step_fused(q, "bf16")
    ref = c.oracle_attend(q)
    err = assert_close(got, ref, "d=168 layer decode")
    log(f"  max abs err {err:.2e}, worst err/tol {err_tol_ratio(got, ref):.4f}")
    c.check_codes(seqs=[0, 7])


def test_int4_d168_unsupported(rt):
    """int4's groups of 32 do not divide 168: the cache refuses it."""
    with pytest.raises(S.SaiError) as e:
        S.KvCache(rt, 1, 8, D, 16, 1, 4, S.KV_INT4)
    assert e.value.kind == "Unsupported"


# ---------------------------------------------------------------- prefill ---
@pytest.mark.parametrize("hq,past,new,qd,interleaved", [
    (32, [300, 0], 150, "bf16", False), (8, [100, 37], 70, "f32", True),
    (64, [64, 640], 33, "f32", False)])
def test_prefill_d168(rt, hq, past, new, qd, interleaved):
    log(f"prefill d=168 hq={hq} past={past} new={new} {qd} interleaved={interleaved}")
    c = Case(rt, 0x1693 + new, len(past), hq, 8, D, past, new, theta=THETA, permute_pages=True,
             kv_dtype=qd, interleaved=interleaved)
    c.step_kv()
    c.check_codes()
    q = c.query(qd)
    got = c.gpu_prefill(q, qd)
    ref = c.oracle_attend(q)
    log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
    assert_close(got, ref, "d=168 prefill")


def test_prefill_d168_outlier_keys_window_bf16_out(rt):
    """x20 outlier channels (Student-t elsewhere), a 64-key sliding window and
    bf16 output."""
    from _gpu_util import bf16_tol_close
    log("prefill d=168 outlier keys + window + bf16 output")
    c = Case(rt, 0x1694, 2, 32, 8, D, [200, 31], 90, theta=THETA, kv_dtype="bf16",
             k_transform=outlier_keys(D, (5, 17, 88, 165)))
    c.step_kv()
    q = c.query("bf16")
    assert_close(c.gpu_prefill(q, "bf16"), c.oracle_attend(q), "d=168 outlier prefill")
    assert_close(c.gpu_prefill(q, "bf16", window=64), c.oracle_attend(q, mask_window=64),
                 "d=168 windowed prefill")
    r = bf16_tol_close(c.gpu_prefill(q, "bf16", out_dtype="bf16"), c.oracle_attend(q),
                       "d=168 prefill bf16 output")
    log(f"  bf16 output: worst err/tol {r:.4f}")


def test_prefill_d168_large_v(rt):
    """V x1e5 with keys at 300-339 scaled x6: the precise pass, checked
    against the weighted bound with kappa 2^-12 as at 128."""
    log("prefill d=168 large V")

    def jump(rng, k):
        if k.shape[1] >= 340:
            k[:, 300:340] *= 6.0
        return k

    c = Case(rt, 0x1695, 2, 32, 8, D, [700, 450], 130, theta=THETA, permute_pages=True,
             k_transform=jump, v_transform=lambda rng, v: v * np.float32(1e5))
    c.step_kv()
    c.check_codes()
    q = c.query("f32")
    got = c.gpu_prefill(q, "f32")
    assert np.isfinite(got).all()
    r = assert_close_weighted(got, c.oracle_attend(q), weighted_abs_v(c, q), 2.0 ** -12,
                              "d=168 prefill, large V")
    log(f"  worst err / weighted bound {r:.4f}")
