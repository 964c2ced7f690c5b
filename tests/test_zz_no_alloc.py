"""sai_gqa_with_cache_noalloc: the fused decode step over the library's fixed
per-GPU scratch instead of the cache's workspace.

Two calls in a row through the C ABI, the second with a smaller input (so the
scratch still holds the first call's contents): each against
sai_gqa_with_cache on an identical cache (same seeded inputs), bit-identical
(the same kernels with the default fixed tile order), against the oracle, and
with the appended token's codes bit-exact. A step whose partials exceed the
scratch is rejected with UNSUPPORTED and leaves the cache as it was.
"""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import Case, assert_close, dev, log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    r = S.Runtime(0)
    yield r
    r.close()


def fused(c, q, k, v, noalloc):
    import torch
    out = torch.zeros((c.batch, 1, c.hq * c.d), dtype=torch.float32, device="cuda")
    step = c.cache.decode_with_cache_noalloc if noalloc else c.cache.decode_with_cache
    step(0, dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16"), out, c.batch, c.hq, c.cos_d,
         c.sin_d, c.cos.shape[0])
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("call", [0, 1])
def test_noalloc_matches_with_cache(rt, call):
    # call 0: a uniform 8 x 4096 batch (two splits each, merged in-kernel);
    # call 1, smaller: a ragged 3-sequence batch at head_dim 64 (combine kernel)
    shapes = [dict(batch=8, hq=32, hkv=8, d=128, past=[4095] * 8),
              dict(batch=3, hq=16, hkv=4, d=64, past=[500, 77, 1200])]
    sh = shapes[call]
    log(f"noalloc call {call}: {sh}")
    seed = 0xA110C + call
    cases = [Case(rt, seed, sh["batch"], sh["hq"], sh["hkv"], sh["d"], sh["past"], 1, theta=5e5,
                  kv_dtype="bf16", permute_pages=True, extra_tokens=1) for _ in range(2)]
    q = [c.query("bf16") for c in cases]
    kv = [c.kv(1) for c in cases]
    assert np.array_equal(q[0], q[1]) and np.array_equal(kv[0][0], kv[1][0])
    want = fused(cases[0], q[0], *kv[0], noalloc=False)
    got = fused(cases[1], q[1], *kv[1], noalloc=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"noalloc differs from with_cache, call {call}: max |diff| {np.abs(got - want).max():.3e}"
    assert_close(got, want, f"noalloc vs with_cache, call {call}")
    c = cases[1]
    c.ocache.append(*kv[1], c.cos, c.sin, c.do_rotary, c.interleaved)
    assert_close(got, c.oracle_attend(q[1]), f"noalloc vs oracle, call {call}")
    c.check_codes(seqs=[0, c.batch - 1])


def test_noalloc_rejects_a_step_beyond_its_scratch(rt):
    """4 x 8192 tokens, 64 query / 8 kv heads, split forced to 64 tokens:
    512 sequence-splits x 8 kv heads x 8 heads x 130 floats = 4,259,840
    partial floats, past the scratch's 4,063,232."""
    log("noalloc: a step beyond the scratch is rejected")
    c = Case(rt, 0xA110F, 4, 64, 8, 128, [8191] * 4, 1, theta=5e5, kv_dtype="bf16",
             extra_tokens=1)
    q = c.query("bf16")
    k, v = c.kv(1)
    prev = rt.set_decode_split(64)
    try:
        with pytest.raises(S.SaiError) as ei:
            fused(c, q, k, v, noalloc=True)
        assert ei.value.status == -3 and "fixed scratch" in str(ei.value), str(ei.value)
    finally:
        rt.set_decode_split(prev)
    assert c.cache.lengths()[1] == 0  # nothing left pending
    # the same step at the automatic split fits, and matches the oracle
    got = fused(c, q, k, v, noalloc=True)
    c.ocache.append(k, v, c.cos, c.sin, c.do_rotary, c.interleaved)
    assert_close(got, c.oracle_attend(q), "noalloc after a rejected step")


def test_noalloc_head168(rt):
    """head_dim 168 (Gemma 4 31B, stored 192 wide): the fixed scratch holds
    the split partials at the stored width; bit-identical to
    sai_gqa_with_cache, within the oracle's tolerance, codes bit-exact."""
    log("noalloc head_dim 168: 4 sequences, 32Q/8KV, ragged")
    past = [3000, 17, 900, 4095]
    cases = [Case(rt, 0xA1168, 4, 32, 8, 168, past, 1, theta=1e6, kv_dtype="bf16",
                  permute_pages=True, extra_tokens=1) for _ in range(2)]
    q = [c.query("bf16") for c in cases]
    kv = [c.kv(1) for c in cases]
    want = fused(cases[0], q[0], *kv[0], noalloc=False)
    got = fused(cases[1], q[1], *kv[1], noalloc=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"noalloc differs from with_cache at head_dim 168: max |diff| {np.abs(got - want).max():.3e}"
    c = cases[1]
    c.ocache.append(*kv[1], c.cos, c.sin, c.do_rotary, c.interleaved)
    assert_close(got, c.oracle_attend(q[1]), "noalloc head_dim 168 vs oracle")
    c.check_codes(seqs=[0, 3])
