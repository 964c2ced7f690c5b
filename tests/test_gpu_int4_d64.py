"""int4 decode at head_dim 64 (two groups of 32 dims per row).

The int4 decode kernel keeps its head_dim-128 column layout (four lane groups,
one per 32-dim group) at 64: lane groups 2 and 3 carry zero query dims and
zero group parameters, so they add nothing, and the split-half RoPE partner is
the lane 16 away. These cases restate the head_dim-128 int4 decode tests at 64:
every GQA group, Student-t keys with x20 outlier channels, permuted pages,
the RoPE/scale/dtype options, forced split merges over ragged lengths, and the
fused append + decode step with codes bit-exact against the oracle.

Reference semantics being matched: scaled_dot_product_attention
(onnx-rt/src/ops/microsoft.rs:241-299, :380-438) over the cache dequantised
with the min/max quantiser (onnx-rt/src/kv_compression.rs:223-253).
"""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import Case, assert_close, err_tol_ratio, log, outlier_keys

pytestmark = pytest.mark.gpu

D = 64
K64 = outlier_keys(D, (5, 17, 40, 61))


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    r = S.Runtime(0)
    yield r
    r.close()


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (16, 2)])
def test_decode_int4_d64_groups(rt, hq, hkv):
    log(f"decode int4 D=64 group {hq // hkv}: hq={hq} hkv={hkv}, outlier K, permuted pages")
    c = Case(rt, 0x6400 + hq, 3, hq, hkv, D, [300, 129, 17], 1, theta=1e4, quant=S.KV_INT4,
             k_transform=K64, permute_pages=True)
    c.step_kv()
    c.check_codes()
    q = c.query()
    got, ref = c.gpu_decode(q), c.oracle_attend(q)
    log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
    assert_close(got, ref, f"int4 D=64 group {hq // hkv}")


def test_decode_int4_d64_options(rt):
    log("decode int4 D=64: no rotary / interleaved / explicit scale / bf16")
    for rot, inter, scale, dt in [(False, False, None, "f32"), (True, True, None, "bf16"),
                                  (True, False, 0.07, "f32")]:
        c = Case(rt, 0x6410, 2, 16, 4, D, [200, 90], 1, quant=S.KV_INT4, do_rotary=rot,
                 interleaved=inter, kv_dtype=dt)
        c.step_kv()
        q = c.query(dt)
        assert_close(c.gpu_decode(q, dt, scale=scale), c.oracle_attend(q, scale),
                     f"int4 D=64 {rot} {inter} {scale} {dt}")


def test_decode_int4_d64_first_token_equals_v(rt):
    log("decode int4 D=64 first token")
    c = Case(rt, 0x6420, 2, 8, 2, D, [0, 0], 1, quant=S.KV_INT4)
    c.step_kv()
    q = c.query()
    got = c.gpu_decode(q)
    _, vd = c.ocache.dequant()
    for b in range(2):
        for hq in range(8):
            np.testing.assert_allclose(got[b, 0, hq * D:(hq + 1) * D], vd[b, hq // 4, 0],
                                       atol=2e-3, rtol=1e-3)


@pytest.mark.parametrize("split", [64, 1024])
def test_decode_int4_d64_split_merge(rt, split):
    log(f"decode int4 D=64 split merge split={split}")
    c = Case(rt, 0x6430, 3, 32, 8, D, [3000, 1, 640], 1, quant=S.KV_INT4, k_transform=K64,
             permute_pages=True)
    prev = rt.set_decode_split(split)
    try:
        c.step_kv()
        q = c.query()
        ref = c.oracle_attend(q)
        for _ in range(2):
            assert_close(c.gpu_decode(q), ref, f"int4 D=64 split {split}")
    finally:
        rt.set_decode_split(prev)


@pytest.mark.parametrize("split", [64, 4096])
def test_decode_int4_d64_fused_step(rt, split):
    """Fused int4 step at head_dim 64: the decode kernel appends the token (V
    nibble shared with the neighbouring slot) and attends; codes bit-exact."""
    log(f"fused int4 D=64 decode step split={split}")
    prev_s = rt.set_decode_split(split)
    try:
        c = Case(rt, 0x6440, 3, 32, 8, D, [700, 4, 4100], 1, theta=1e4, kv_dtype="bf16",
                 quant=S.KV_INT4, k_transform=K64, permute_pages=True, extra_tokens=2)
        for step in range(3):
            q = c.query("bf16")
            got = c.step_fused(q, "bf16")
            assert_close(got, c.oracle_attend(q), f"fused int4 D=64 step {step}")
            c.check_codes(seqs=[1])
            c.cache.advance()
    finally:
        rt.set_decode_split(prev_s)


@pytest.mark.parametrize("lw,w", [(0, 100), (300, 0), (70, 33)])
def test_decode_int4_d64_window(rt, lw, w):
    """Sliding windows over the int4 D=64 cache: a sliding layer (its last lw
    keys), the mask rule of local_window_size, and both at once."""
    log(f"decode int4 D=64 window layer_window={lw} window={w}")
    c = Case(rt, 0x6450 + lw + w, 3, 16, 4, D, [900, 150, 64], 1, quant=S.KV_INT4,
             k_transform=K64, permute_pages=True)
    c.cache.set_layer_window(0, lw)
    c.step_kv()
    q = c.query()
    got = c.gpu_decode(q, window=w)
    assert_close(got, c.oracle_attend(q, layer_window=lw, mask_window=w),
                 f"int4 D=64 lw={lw} w={w}")
