"""Sliding windows on the GPU against the oracle, through the C ABI.

Two reference rules, as in oracle/sai_oracle.c first_visible_key:
* `window` (the node's local_window_size; gpu_gqa_with_cache's window and the
  mask of cuda/kernels/attention.rs:79): the query at position p sees keys
  [p - window, p];
* a sliding-window cache layer (sai_kvcache_set_layer_window; GpuKvCache::view_at,
  cuda/kv_cache.rs:340-360): the query sees its last w keys.
Decode (int8 and int4, separate and fused append, one and many splits,
ragged lengths shorter and longer than the window) and prefill (int8 and
int4). Bar: outputs within 2e-3 abs + 1e-2 rel of the oracle, which attends
over the same dequantised cache.
"""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import Case, assert_close, log, outlier_student_t

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    assert S.lib().sai_device_supported(0) == 1, "device 0 is not gfx950"
    r = S.Runtime(0)
    yield r
    r.close()


DECODE = [
    # (layer_window, window): node window only, layer window only, both, tiny
    (0, 100), (256, 0), (100, 300), (300, 100), (1, 0), (0, 1), (64, 0), (0, 63), (5000, 0),
]


@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
@pytest.mark.parametrize("lw,w", DECODE)
def test_decode_window_ragged(rt, quant, lw, w):
    log(f"decode window quant={quant} layer_window={lw} window={w}")
    lens = [1000, 37, 255, 256, 700, 1, 129, 2048]
    c = Case(rt, 900 + lw + w, len(lens), 16, 4, 128, lens, 1, theta=5e5, quant=quant,
             permute_pages=True,
             k_transform=outlier_student_t if quant == S.KV_INT4 else None)
    c.cache.set_layer_window(0, lw)
    c.step_kv()
    q = c.query("bf16")
    got = c.gpu_decode(q, "bf16", window=w)
    ref = c.oracle_attend(q, layer_window=lw, mask_window=w)
    assert_close(got, ref, f"decode lw={lw} w={w}")


@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
@pytest.mark.parametrize("split", [0, 256])
def test_decode_window_many_splits_fused(rt, quant, split):
    """Long contexts cut into many splits (split 256 forced) with the window's
    first key inside a split's first tile; the fused append writes the token."""
    log(f"decode window many splits quant={quant} split={split}")
    lens = [9000, 7001, 12345]
    c = Case(rt, 950 + split, len(lens), 32, 8, 128, lens, 0, theta=5e5, quant=quant,
             extra_tokens=1)
    prev = rt.set_decode_split(split)
    try:
        for lw, w in ((0, 3000), (2500, 0), (1000, 777)):
            c.cache.set_layer_window(0, lw)
            q = c.rng.standard_normal((c.batch, 1, c.hq * c.d), dtype=np.float32)
            got = c.step_fused(q, window=w)
            ref = c.oracle_attend(q, layer_window=lw, mask_window=w)
            assert_close(got, ref, f"fused lw={lw} w={w}")
            c.check_codes()
            # back to the committed state for the next pair (same slot rewritten)
            c.ocache.seq_len = c.ocache.seq_len - 1
    finally:
        rt.set_decode_split(prev)


@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
@pytest.mark.parametrize("lw,w", [(0, 64), (100, 0), (0, 200), (33, 70), (1, 0), (0, 1000)])
def test_prefill_window(rt, quant, lw, w):
    log(f"prefill window quant={quant} layer_window={lw} window={w}")
    past = [300, 0, 517]
    c = Case(rt, 970 + lw + w, len(past), 8, 2, 128, past, 200, theta=5e5, quant=quant,
             permute_pages=True, kv_dtype="bf16")
    c.cache.set_layer_window(0, lw)
    c.step_kv()
    q = c.query("bf16")
    got = c.gpu_prefill(q, "bf16", window=w)
    ref = c.oracle_attend(q, layer_window=lw, mask_window=w)
    assert_close(got, ref, f"prefill lw={lw} w={w}")


def test_layer_window_errors(rt):
    c = Case(rt, 5, 1, 4, 1, 64, [10], 1)
    with pytest.raises(S.SaiError) as e:
        c.cache.set_layer_window(3, 4)
    assert e.value.kind == "ShapeMismatch"
    with pytest.raises(S.SaiError) as e:
        c.cache.set_layer_window(0, -1)
    assert e.value.kind == "InvalidAttribute"
