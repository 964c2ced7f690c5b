"""The decode step, the prefill and the TurboQuant step captured in a HIP graph
(torch.cuda.graph over the C ABI calls) and replayed.

A serving loop may capture its per-token launches once and replay them. Every
entry point here launches its kernels with parameters passed by value and
clears nothing with memset nodes (split-merge tickets reset themselves in the
kernel), so a captured step replays the eager step exactly. Each graph is
replayed four times with eager work and synchronisations between the replays,
and every replay must equal the eager result bit for bit (fixed tile orders).
The step's inputs (lengths, the pending token's slot) do not change between
replays; a graph captured for one set of lengths is only valid for those.
"""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import Case, dev, log, to_bf16_f32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    assert S.lib().sai_device_supported(0) == 1, "device 0 is not gfx950"
    r = S.Runtime(0)
    yield r
    r.close()


def replay_matches(step, out, reps=4):
    """Eager result, then the captured step replayed `reps` times with eager
    work (a fill of the output, an unrelated product) between replays."""
    import torch
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        step(s)
    torch.cuda.synchronize()
    ref = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        step(s)
    torch.cuda.synchronize()
    scratch = torch.randn(256, 256, device="cuda")
    for r in range(reps):
        out.fill_(float("nan"))
        scratch = scratch @ scratch.t() * 1e-3
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r} differs from the eager step"
    return ref


@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
@pytest.mark.parametrize("split", [0, 256])
def test_fused_decode_step_graph(rt, quant, split):
    """sai_gqa_with_cache (append + decode + in-kernel merge) in a graph; the
    replays rewrite the same pending slot."""
    import torch
    log(f"graph: fused decode quant={quant} split={split}")
    lens = [700, 1500, 33]
    c = Case(rt, 0x6A0 + quant + split, len(lens), 16, 4, 128, lens, 0, quant=quant,
             permute_pages=True, extra_tokens=1)
    prev = rt.set_decode_split(split)
    try:
        q = c.rng.standard_normal((c.batch, 1, c.hq * c.d), dtype=np.float32)
        k, v = c.kv(1)
        qd, kd, vd = dev(q, "bf16"), dev(k), dev(v)
        out = torch.zeros((c.batch, 1, c.hq * c.d), device="cuda")

        def step(s):
            c.cache.decode_with_cache(0, qd, kd, vd, out, c.batch, c.hq, c.cos_d, c.sin_d,
                                      c.cos.shape[0], c.do_rotary, c.interleaved, stream=s)

        got = replay_matches(step, out)
        c.ocache.append(k, v, c.cos, c.sin, c.do_rotary, c.interleaved)
        ref = c.oracle_attend(to_bf16_f32(q))
        assert np.allclose(got.cpu().numpy(), ref, atol=2e-3, rtol=1e-2)
    finally:
        rt.set_decode_split(prev)


def test_prefill_graph(rt):
    """The prefill (fast pass and the precise pass's flag check) in a graph."""
    import torch
    log("graph: prefill")
    c = Case(rt, 0x6B0, 2, 16, 4, 128, [300, 0], 130, permute_pages=True)
    c.step_kv()
    q = c.query()
    qd = dev(q)
    out = torch.zeros((c.batch, c.new_tokens, c.hq * c.d), device="cuda")

    def step(s):
        c.cache.prefill(0, qd, out, c.batch, c.new_tokens, c.hq, c.cos_d, c.sin_d, c.cos.shape[0],
                        c.do_rotary, c.interleaved, stream=s)

    got = replay_matches(step, out)
    ref = c.oracle_attend(q)
    assert np.allclose(got.cpu().numpy(), ref, atol=2e-3, rtol=1e-2)


def test_turboquant_step_graph(rt):
    """sai_tqcache_write_attend (store + attention + merge + rotation back) in a
    graph, with the fixed tile order."""
    import torch
    log("graph: turboquant write_attend")
    d, bits, heads, group = 128, 4, 2, 4
    lens = [900, 4100]
    batch, nh = len(lens), heads * group
    rng = np.random.default_rng(0x6C0)
    prev = rt.set_decode_reproducible(1)
    c = S.TqCache(rt, 1, heads, d, bits, True, batch, max(lens) + 1, seed=11)
    try:
        k0 = torch.from_numpy(rng.standard_normal((batch, max(lens), heads * d)).astype(np.float32)).cuda()
        v0 = torch.from_numpy(rng.standard_normal((batch, max(lens), heads * d)).astype(np.float32)).cuda()
        c.write(0, k0, v0, batch, max(lens))
        c.advance()
        c.set_lengths(lens)
        q = torch.from_numpy(rng.standard_normal((batch, 1, nh * d)).astype(np.float32)).cuda()
        kn = torch.from_numpy(rng.standard_normal((batch, 1, heads * d)).astype(np.float32)).cuda()
        vn = torch.from_numpy(rng.standard_normal((batch, 1, heads * d)).astype(np.float32)).cuda()
        out = torch.zeros((batch, 1, nh * d), device="cuda")

        def step(s):
            c.write_attend(0, q, kn, vn, out, batch, nh, stream=s)

        got = replay_matches(step, out)
        assert torch.isfinite(got).all()
    finally:
        c.close()
        rt.set_decode_reproducible(prev)
