"""Caches of one context used from several streams.

Each cache owns the device scratch of its attention launches (split partials,
split ranges, merge tickets), so two caches may decode at the same time on two
streams of one sai_ctx; launches on one cache stay ordered on its stream. The
calls documented as synchronous (reads, reset) wait for work enqueued on any
stream first. The reference holds its cache behind a mutex and runs one
stream (onnx-rt/src/session.rs:377); these cases pin the stream model this
boundary documents instead.
"""
import numpy as np
import pytest

import oracle as O
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


def test_two_caches_two_streams(rt):
    """Interleaved fused decode steps (append + attend + advance) on two
    int8 caches of different shapes, each on its own stream, both checked
    against the oracle step by step; the ragged one merges in the combine
    kernel, the uniform one in-kernel (automatic merge)."""
    import torch
    log("two caches, two streams: 3 fused steps each, interleaved")
    a = Case(rt, 0x5711, 4, 32, 8, 128, [3000, 700, 129, 2048], 1, theta=5e5,
             kv_dtype="bf16", permute_pages=True, extra_tokens=3)
    b = Case(rt, 0x5712, 8, 16, 2, 128, [4095] * 8, 1, theta=5e5, kv_dtype="bf16",
             extra_tokens=3)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs, refs = {"a": [], "b": []}, {"a": [], "b": []}
    for step in range(3):
        for name, c, s in (("a", a, s1), ("b", b, s2)):
            q = c.query("bf16")
            k, v = c.kv(1)
            c.ocache.append(k, v, c.cos, c.sin, c.do_rotary, c.interleaved)
            refs[name].append(c.oracle_attend(q))
            qd, kd, vd = dev(q, "bf16"), dev(k, "bf16"), dev(v, "bf16")
            torch.cuda.synchronize()  # inputs resident before the streams run
            out = torch.zeros((c.batch, 1, c.hq * c.d), dtype=torch.float32, device="cuda")
            with torch.cuda.stream(s):
                c.cache.decode_with_cache(0, qd, kd, vd, out, c.batch, c.hq, c.cos_d, c.sin_d,
                                          c.cos.shape[0], stream=s)
                c.cache.advance(stream=s)
            outs[name].append((out, qd, kd, vd))
    torch.cuda.synchronize()
    for name in ("a", "b"):
        for step, ((out, *_), ref) in enumerate(zip(outs[name], refs[name])):
            assert_close(out.cpu().numpy(), ref, f"cache {name} step {step}")
    a.check_codes(seqs=[2])
    b.check_codes(seqs=[5])


def test_tq_side_stream_then_synchronous_read_and_reset(rt):
    """TurboQuant rows written and attended on a side stream are what the
    synchronous read returns right after (no caller synchronisation), and a
    synchronous reset after queued work leaves an empty cache."""
    import torch
    log("tq cache: write + attend on a side stream, then read / reset")
    d, bits, heads, group, batch, rows = 128, 4, 2, 4, 2, 300
    rng = np.random.default_rng(99)
    c = S.TqCache(rt, 1, heads, d, bits, True, batch, rows + 1, seed=7)
    try:
        k = rng.standard_normal((batch, rows, heads * d)).astype(np.float32)
        v = rng.standard_normal((batch, rows, heads * d)).astype(np.float32)
        q = rng.standard_normal((batch, 1, heads * group * d)).astype(np.float32)
        kd, vd, qd = dev(k), dev(v), dev(q)
        out = torch.zeros((batch, 1, heads * group * d), device="cuda")
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            c.write(0, kd, vd, batch, rows, stream=s)
            c.advance(stream=s)
            c.attend(0, qd, out, batch, heads * group, stream=s)
        # synchronous read straight after the side stream's launches
        kr, vr = c.read(0, 1, 1, 0, rows)
        sg = O.tq_signs(O.tq_head_seed(7, 0, heads, 1), d)
        rk = np.ascontiguousarray(k[1].reshape(rows, heads, d)[:, 1])
        rv = np.ascontiguousarray(v[1].reshape(rows, heads, d)[:, 1])
        ek = O.tq_write_rows(rk, bits, sg, True)
        ev = O.tq_write_rows(rv, bits, sg, True)
        for t in (0, 137, rows - 1):
            wk = O.tq_decode(ek[0][t], d, bits, ek[1][t], ek[2][t], sg)
            wv = O.tq_decode(ev[0][t], d, bits, ev[1][t], ev[2][t], sg)
            assert np.array_equal(kr[t].view(np.uint32), wk.view(np.uint32)), t
            assert np.array_equal(vr[t].view(np.uint32), wv.view(np.uint32)), t
        s.synchronize()
        want = O.tq_attend(q[1, 0].reshape(heads * group, d)[group:2 * group], bits, True, sg, ek,
                           ev, S.default_scale(d))
        got = out.cpu().numpy()[1, 0].reshape(heads * group, d)[group:2 * group]
        np.testing.assert_allclose(got, want, atol=2e-3, rtol=1e-2)
        # queue more work on the side stream, then reset synchronously
        with torch.cuda.stream(s):
            c.write(0, kd[:, :1].contiguous(), vd[:, :1].contiguous(), batch, 1, stream=s)
        c.reset()
        lens, pending, _ = c.lengths()
        assert list(lens[:batch]) == [0, 0] and pending == 0
    finally:
        c.close()
