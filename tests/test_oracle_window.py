"""Pins of the oracle's window rules (oracle/sai_oracle.c first_visible_key,
sai_or_sdpa_window, sai_or_gqa_cached_window).

The reference has two rules and a test for each, restated here:
* the GPU softmax mask (cuda/kernels/attention.rs:79, :111): a query at
  q_pos sees keys [q_pos - window, q_pos]; test_gpu_masked_softmax_sliding_window
  (tests/test_cuda.rs:3157-3200: window 4 over 16 x 16, out-of-window weights
  0, rows summing to 1);
* a sliding-window cache layer (cuda/kv_cache.rs:340-360): the view after
  appending holds the last w keys; test_kv_cache_sliding_window
  (test_cuda.rs:1275-1334: 6 tokens, window 4, the view is positions 2..5).
With V the identity matrix the attention output row is the softmax weight row,
so both become exact statements about which weights are zero. Closed forms
beside them: a span of one key returns that key's V exactly; a window at least
as long as the sequence changes nothing (bit for bit); both rules together
take the narrower; an f64 brute force over random data.
"""
import numpy as np
import pytest

import oracle as O


def weights(sq, sk, past, layer_window=0, mask_window=0, seed=0):
    """Softmax weight rows [Sq, Sk] of one head, read through V = I."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((1, 1, sq, sk)).astype(np.float32)
    k = rng.standard_normal((1, 1, sk, sk)).astype(np.float32)
    v = np.eye(sk, dtype=np.float32)[None, None]
    return O.sdpa_window(q, k, v, 1, past, 0.3, layer_window, mask_window)[0, 0]


def test_reference_mask_window_kat():
    # test_cuda.rs:3157-3200: q_pos attends to [q_pos - 4, q_pos]
    w = weights(16, 16, 0, mask_window=4)
    for qi in range(16):
        for kj in range(16):
            allowed = kj <= qi and kj >= qi - 4
            if not allowed:
                assert w[qi, kj] == 0.0, (qi, kj)
            else:
                assert w[qi, kj] > 0.0, (qi, kj)
        assert abs(w[qi].sum() - 1.0) < 1e-5
    # the reference's examples: q=0 -> {0}, q=5 -> {1..5}, q=15 -> {11..15}
    assert np.flatnonzero(w[0]).tolist() == [0]
    assert np.flatnonzero(w[5]).tolist() == [1, 2, 3, 4, 5]
    assert np.flatnonzero(w[15]).tolist() == list(range(11, 16))


def test_reference_cache_layer_window_kat():
    # test_cuda.rs:1275-1334: 6 tokens, window 4 -> the view is positions 2..5;
    # one decode query at position 5 attends to exactly those
    w = weights(1, 6, 5, layer_window=4)
    assert np.flatnonzero(w[0]).tolist() == [2, 3, 4, 5]
    assert abs(w[0].sum() - 1.0) < 1e-5
    # while the global layer sees all 6
    g = weights(1, 6, 5)
    assert np.flatnonzero(g[0]).tolist() == list(range(6))


def test_span_of_one_returns_that_value_exactly():
    rng = np.random.default_rng(1)
    sq, sk, past, d = 5, 12, 7, 16
    q = rng.standard_normal((1, 2, sq, d)).astype(np.float32)
    k = rng.standard_normal((1, 1, sk, d)).astype(np.float32)
    v = rng.standard_normal((1, 1, sk, d)).astype(np.float32)
    for kwargs in (dict(layer_window=1), dict(mask_window=0, layer_window=1)):
        out = O.sdpa_window(q, k, v, 1, past, 0.2, **kwargs)
        for qi in range(sq):
            assert np.array_equal(out[0, :, qi], np.broadcast_to(v[0, 0, past + qi], (2, d)))
    # mask window 0 is off, not "one key"
    out = O.sdpa_window(q, k, v, 1, past, 0.2, mask_window=0)
    assert np.array_equal(out, O.sdpa(q, k, v, 1, past, 0.2, True))


def test_long_windows_change_nothing():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((2, 4, 6, 32)).astype(np.float32)
    k = rng.standard_normal((2, 2, 40, 32)).astype(np.float32)
    v = rng.standard_normal((2, 2, 40, 32)).astype(np.float32)
    ref = O.sdpa(q, k, v, 2, 34, 0.17, True)
    assert np.array_equal(O.sdpa_window(q, k, v, 2, 34, 0.17, layer_window=40), ref)
    assert np.array_equal(O.sdpa_window(q, k, v, 2, 34, 0.17, mask_window=39), ref)
    assert not np.array_equal(O.sdpa_window(q, k, v, 2, 34, 0.17, layer_window=39), ref)


@pytest.mark.parametrize("lw,mw", [(5, 0), (0, 5), (5, 2), (3, 7), (9, 9)])
def test_windows_against_f64_brute_force(lw, mw):
    rng = np.random.default_rng(lw * 10 + mw)
    b, hq, hk, sq, past, d = 2, 4, 2, 7, 13, 16
    sk = past + sq
    q = rng.standard_normal((b, hq, sq, d)).astype(np.float32)
    k = rng.standard_normal((b, hk, sk, d)).astype(np.float32)
    v = rng.standard_normal((b, hk, sk, d)).astype(np.float32)
    got = O.sdpa_window(q, k, v, hk, past, 0.25, lw, mw)
    want = np.zeros((b, hq, sq, d))
    for bi in range(b):
        for h in range(hq):
            kh = h // (hq // hk)
            for qi in range(sq):
                p = past + qi
                lo = 0
                if mw > 0:
                    lo = max(lo, p - mw)
                if lw > 0:
                    lo = max(lo, p + 1 - lw)
                keys = np.arange(lo, p + 1)
                s = (k[bi, kh, keys].astype(np.float64) @ q[bi, h, qi].astype(np.float64)) * 0.25
                e = np.exp(s - s.max())
                want[bi, h, qi] = (e / e.sum()) @ v[bi, kh, keys].astype(np.float64)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=1e-4)


def test_cached_gqa_window_matches_sdpa_window():
    """sai_or_gqa_cached_window over a dequantised int8 cache equals
    sdpa_window on the same (dequantised, RoPE-rotated) keys."""
    rng = np.random.default_rng(4)
    b, hkv, hq, d, past, sq = 2, 2, 4, 64, 30, 3
    cos, sin = O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.ones((64, 32), np.float32))), \
        np.zeros((64, 32), np.float32)
    lc = O.LogicalCache(b, hkv, d, past + sq)
    lc.append(rng.standard_normal((b, past, hkv * d)), rng.standard_normal((b, past, hkv * d)),
              cos, sin)
    lc.append(rng.standard_normal((b, sq, hkv * d)), rng.standard_normal((b, sq, hkv * d)),
              cos, sin)
    qv = rng.standard_normal((b, sq, hq * d)).astype(np.float32)
    kd, vd = lc.dequant()
    for lw, mw in ((0, 0), (6, 0), (0, 4), (8, 3)):
        got = lc.attend(qv, hq, cos, sin, layer_window=lw, mask_window=mw)
        qb = qv.reshape(b, sq, hq, d).transpose(0, 2, 1, 3)  # identity RoPE (cos 1, sin 0)
        want = O.sdpa_window(qb, kd, vd, hkv, past, O.lib().sai_or_default_scale(d), lw, mw)
        assert np.array_equal(got, want.transpose(0, 2, 1, 3).reshape(b, sq, hq * d)), (lw, mw)
