"""The TurboQuant compressed KV cache on the GPU (sai_tqcache_*), against the
oracle's restatement of CompressedKVCache (onnx-rt/src/kv_compression.rs:
738-963) and of the decode read path over it.

Stored form (codes, scale, zero point, QJL sign bits and mean) is checked bit
for bit against oracle.tq_write_rows with the cache's per-head seeds; decoded
rows (read_k / read_v) bit for bit against oracle.tq_decode; attention
against oracle.tq_attend within 2e-3 abs + 1e-2 rel (the kernel evaluates
the same estimator in the rotated domain, so only rounding differs)."""
import numpy as np
import pytest

import oracle as O
import smallaios_amd as S
from _gpu_util import log

pytestmark = pytest.mark.gpu
SEED = 0xDEADBEEFCAFE1234


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    r = S.Runtime(0)
    yield r
    r.close()


def head_signs(seed, layer, heads, h, d):
    return O.tq_signs(O.tq_head_seed(seed, layer, heads, h), d)


def rows_of(x, b, h, heads, d):
    """Rows of (sequence b, kv head h) from host [B, S, heads*D] f32."""
    return np.ascontiguousarray(x[b].reshape(x.shape[1], heads, d)[:, h])


def to_dev(x, bf16):
    import torch
    t = torch.from_numpy(x)
    return (t.to(torch.bfloat16) if bf16 else t).cuda()


def host_vals(x, bf16):
    """The f32 values the kernel reads from the device copy of x."""
    if not bf16:
        return x
    return O.bf16_bits_to_f32(O.f32_to_bf16_bits(x)).reshape(x.shape)


def check_rows(cache, layer, b, h, t0, x_k, x_v, heads, d, bits, qjl, seed):
    n = x_k.shape[0]
    sg = head_signs(seed, layer, heads, h, d)
    raw = cache.read_raw(layer, b, h, t0, n)
    for kind, x in (("k", x_k), ("v", x_v)):
        codes, sc, z, sb, c = O.tq_write_rows(x, bits, sg, qjl)
        assert np.array_equal(raw[f"{kind}_codes"], codes), (kind, b, h)
        assert np.array_equal(raw[f"{kind}_params"][:, 0].view(np.uint32), sc.view(np.uint32))
        assert np.array_equal(raw[f"{kind}_params"][:, 1].view(np.uint32), z.view(np.uint32))
        if qjl:
            assert np.array_equal(raw[f"{kind}_signs"], sb), (kind, b, h)
            assert np.array_equal(raw[f"{kind}_params"][:, 2].view(np.uint32), c.view(np.uint32))
    dk, dv = cache.read(layer, b, h, t0, n)
    ek = O.tq_write_rows(x_k, bits, sg, qjl)
    ev = O.tq_write_rows(x_v, bits, sg, qjl)
    for t in range(n):
        wk = O.tq_decode(ek[0][t], d, bits, ek[1][t], ek[2][t], sg)
        wv = O.tq_decode(ev[0][t], d, bits, ev[1][t], ev[2][t], sg)
        assert np.array_equal(dk[t].view(np.uint32), wk.view(np.uint32)), (b, h, t)
        assert np.array_equal(dv[t].view(np.uint32), wv.view(np.uint32)), (b, h, t)


@pytest.mark.parametrize("d,bits,qjl,bf16", [(128, 4, True, False), (128, 3, True, True),
                                             (64, 8, False, False), (64, 4, True, True),
                                             (128, 8, True, False), (64, 3, False, False),
                                             (256, 4, True, True), (256, 3, True, False),
                                             (256, 8, False, False)])
def test_write_read_bit_exact(rt, d, bits, qjl, bf16):
    """A prefill pass then a decode pass, two layers; every stored row of
    layer 1 checked."""
    import torch
    log(f"tq write/read d={d} bits={bits} qjl={qjl} bf16={bf16}")
    rng = np.random.default_rng(d * 10 + bits)
    batch, heads, s0 = 3, 2, 5
    c = S.TqCache(rt, 2, heads, d, bits, qjl, 4, 16, seed=SEED)
    try:
        passes = []
        for s in (s0, 1):
            ks = [(rng.standard_normal((batch, s, heads * d)) * 0.7).astype(np.float32)
                  for _ in range(2)]
            vs = [(rng.standard_normal((batch, s, heads * d)) * 1.3).astype(np.float32)
                  for _ in range(2)]
            for layer in range(2):
                c.write(layer, to_dev(ks[layer], bf16), to_dev(vs[layer], bf16), batch, s)
            c.advance()
            passes.append((host_vals(ks[1], bf16), host_vals(vs[1], bf16)))
        torch.cuda.synchronize()
        lens, pend, nb = c.lengths()
        assert list(lens[:batch]) == [s0 + 1] * batch and pend == 0 and nb == batch
        for b in range(batch):
            for h in range(heads):
                xk = np.concatenate([rows_of(p[0], b, h, heads, d) for p in passes])
                xv = np.concatenate([rows_of(p[1], b, h, heads, d) for p in passes])
                check_rows(c, 1, b, h, 0, xk, xv, heads, d, bits, qjl, SEED)
    finally:
        c.close()


@pytest.mark.parametrize("d,bits", [(128, 3), (64, 4), (128, 8), (256, 4)])
def test_writes_across_tile_boundaries(rt, d, bits):
    """Passes of 70, 1, 130 and 1 rows from unaligned starts: the V tiles
    are read-modify-written by their owning wave at both ends of a pass, and
    the rows already there must survive. Every row checked bit for bit, and
    attention over the result."""
    import torch
    log(f"tq tile boundaries d={d} bits={bits}")
    rng = np.random.default_rng(d + bits)
    batch, heads = 2, 2
    c = S.TqCache(rt, 1, heads, d, bits, True, batch, 256, seed=SEED)
    try:
        ks, vs = [], []
        for s in (70, 1, 130, 1):
            k = rng.standard_normal((batch, s, heads * d)).astype(np.float32)
            v = rng.standard_normal((batch, s, heads * d)).astype(np.float32)
            c.write(0, to_dev(k, False), to_dev(v, False), batch, s)
            c.advance()
            ks.append(k)
            vs.append(v)
        torch.cuda.synchronize()
        k = np.concatenate(ks, axis=1)
        v = np.concatenate(vs, axis=1)
        assert list(c.lengths()[0][:batch]) == [202] * batch
        for b in range(batch):
            for h in range(heads):
                check_rows(c, 0, b, h, 0, rows_of(k, b, h, heads, d), rows_of(v, b, h, heads, d),
                           heads, d, bits, True, SEED)
        nh = heads * 4
        q = rng.standard_normal((batch, 1, nh * d)).astype(np.float32)
        out = torch.zeros((batch, 1, nh * d), device="cuda")
        c.attend(0, to_dev(q, False), out, batch, nh)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(batch, nh, d)
        for b in range(batch):
            for h in range(heads):
                sg = head_signs(SEED, 0, heads, h, d)
                want = oracle_attend(rows_of(k, b, h, heads, d), rows_of(v, b, h, heads, d),
                                     q.reshape(batch, nh, d)[b, 4 * h:4 * h + 4], bits, True, sg,
                                     S.default_scale(d))
                np.testing.assert_allclose(got[b, 4 * h:4 * h + 4], want, atol=2e-3, rtol=1e-2)
    finally:
        c.close()


def test_constant_and_edge_rows(rt):
    """Constant rows (range 0: scale 1.0), zeros, large magnitudes."""
    import torch
    d, heads = 64, 1
    c = S.TqCache(rt, 1, heads, d, 4, True, 1, 8, seed=0)
    try:
        x = np.stack([np.full(d, 3.14, np.float32), np.zeros(d, np.float32),
                      (np.arange(d, dtype=np.float32) - 32) * np.float32(1e4),
                      np.where(np.arange(d) % 2 == 0, 1.0, -1.0).astype(np.float32)])
        k = x.reshape(1, 4, d)
        c.write(0, to_dev(k, False), to_dev(k[:, ::-1].copy(), False), 1, 4)
        torch.cuda.synchronize()
        check_rows(c, 0, 0, 0, 0, x, x[::-1].copy(), heads, d, 4, True, 0)
    finally:
        c.close()


def oracle_attend(cache_rows_k, cache_rows_v, q, bits, qjl, sg, scale):
    ek = O.tq_write_rows(cache_rows_k, bits, sg, qjl)
    ev = O.tq_write_rows(cache_rows_v, bits, sg, qjl)
    return O.tq_attend(q, bits, qjl, sg, ek, ev, scale)


@pytest.mark.parametrize("d,bits,qjl,group,bf16", [
    (128, 4, True, 4, False), (128, 3, True, 8, True), (64, 8, False, 2, False),
    (128, 8, True, 1, False), (64, 4, True, 8, True), (64, 3, False, 4, False),
    (256, 4, True, 2, True), (256, 3, False, 4, False), (256, 8, True, 1, False)])
def test_attend_matches_oracle(rt, d, bits, qjl, group, bf16):
    """Prefill 40 rows, then a decode pass whose appended row is attended
    while pending (one split)."""
    import torch
    log(f"tq attend d={d} bits={bits} qjl={qjl} G={group} bf16={bf16}")
    rng = np.random.default_rng(bits * 100 + group)
    batch, heads, s0 = 2, 2, 40
    nh = heads * group
    c = S.TqCache(rt, 1, heads, d, bits, qjl, batch, 64, seed=SEED)
    try:
        k0 = rng.standard_normal((batch, s0, heads * d)).astype(np.float32)
        v0 = rng.standard_normal((batch, s0, heads * d)).astype(np.float32)
        c.write(0, to_dev(k0, bf16), to_dev(v0, bf16), batch, s0)
        c.advance()
        k1 = rng.standard_normal((batch, 1, heads * d)).astype(np.float32)
        v1 = rng.standard_normal((batch, 1, heads * d)).astype(np.float32)
        c.write(0, to_dev(k1, bf16), to_dev(v1, bf16), batch, 1)
        q = rng.standard_normal((batch, 1, nh * d)).astype(np.float32)
        out = torch.full((batch, 1, nh * d), float("nan"), device="cuda")
        c.attend(0, to_dev(q, bf16), out, batch, nh)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(batch, nh, d)
        kk = np.concatenate([host_vals(k0, bf16), host_vals(k1, bf16)], axis=1)
        vv = np.concatenate([host_vals(v0, bf16), host_vals(v1, bf16)], axis=1)
        qq = host_vals(q, bf16).reshape(batch, nh, d)
        scale = S.default_scale(d)
        for b in range(batch):
            for h in range(heads):
                sg = head_signs(SEED, 0, heads, h, d)
                want = oracle_attend(rows_of(kk, b, h, heads, d), rows_of(vv, b, h, heads, d),
                                     qq[b, h * group:(h + 1) * group], bits, qjl, sg, scale)
                np.testing.assert_allclose(got[b, h * group:(h + 1) * group], want,
                                           atol=2e-3, rtol=1e-2)
    finally:
        c.close()


def test_attend_long_ragged_splits(rt):
    """Ragged lengths over several 1024-row splits (one sequence shorter than
    a split, one ending mid-tile), explicit scale."""
    import torch
    log("tq attend ragged long")
    d, bits, qjl, group, heads = 128, 4, True, 4, 2
    nh = heads * group
    lens = [3000, 700, 2049]
    batch, rows = len(lens), max(lens)
    rng = np.random.default_rng(11)
    c = S.TqCache(rt, 1, heads, d, bits, qjl, batch, rows, seed=7)
    try:
        k = rng.standard_normal((batch, rows, heads * d)).astype(np.float32)
        v = rng.standard_normal((batch, rows, heads * d)).astype(np.float32)
        c.write(0, to_dev(k, False), to_dev(v, False), batch, rows)
        c.advance()
        c.set_lengths(lens)
        q = (rng.standard_normal((batch, 1, nh * d)) * 2.0).astype(np.float32)
        out = torch.zeros((batch, 1, nh * d), device="cuda")
        c.attend(0, to_dev(q, False), out, batch, nh, scale=0.05)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(batch, nh, d)
        qq = q.reshape(batch, nh, d)
        for b in range(batch):
            for h in range(heads):
                sg = head_signs(7, 0, heads, h, d)
                want = oracle_attend(rows_of(k, b, h, heads, d)[:lens[b]],
                                     rows_of(v, b, h, heads, d)[:lens[b]],
                                     qq[b, h * group:(h + 1) * group], bits, qjl, sg, 0.05)
                np.testing.assert_allclose(got[b, h * group:(h + 1) * group], want,
                                           atol=2e-3, rtol=1e-2)
    finally:
        c.close()


@pytest.mark.parametrize("d,bits,qjl,group", [(128, 4, True, 4), (64, 8, False, 8),
                                               (128, 3, True, 2), (256, 4, True, 4)])
def test_logits_and_weighted_sum(rt, d, bits, qjl, group):
    """The design's attention_logits and weighted_value_sum over ragged
    sequences (two splits for one of them). Logits: the integer-exact path
    differs from the oracle's f32 dot by rounding only. Weighted sum: each
    weight enters the f16 product with a relative error of at most 2^-11, so
    |error| <= 2^-11 * sum_t |w_t| |decode(v_t)| (plus f32 rounding)."""
    import torch
    log(f"tq logits/wsum d={d} bits={bits} qjl={qjl} G={group}")
    rng = np.random.default_rng(bits * 7 + group)
    heads = 2
    nh = heads * group
    lens = [1500, 300]
    batch, rows, ld = len(lens), max(lens), 1536
    c = S.TqCache(rt, 1, heads, d, bits, qjl, batch, rows, seed=SEED)
    try:
        k = rng.standard_normal((batch, rows, heads * d)).astype(np.float32)
        v = rng.standard_normal((batch, rows, heads * d)).astype(np.float32)
        c.write(0, to_dev(k, False), to_dev(v, False), batch, rows)
        c.advance()
        c.set_lengths(lens)
        q = rng.standard_normal((batch, 1, nh * d)).astype(np.float32)
        lg = torch.full((batch * nh, ld), float("nan"), device="cuda")
        c.attention_logits(0, to_dev(q, False), lg, ld, batch, nh)
        w = (rng.random((batch * nh, ld)) * 2 - 1).astype(np.float32)
        out = torch.zeros((batch, 1, nh * d), device="cuda")
        c.weighted_value_sum(0, to_dev(w, False), ld, out, batch, nh)
        torch.cuda.synchronize()
        lg = lg.cpu().numpy().reshape(batch, nh, ld)
        got = out.cpu().numpy().reshape(batch, nh, d)
        qq = q.reshape(batch, nh, d)
        w = w.reshape(batch, nh, ld)
        for b in range(batch):
            n = lens[b]
            assert np.isnan(lg[b, :, n:]).all()
            for h in range(heads):
                sg = head_signs(SEED, 0, heads, h, d)
                ek = O.tq_write_rows(rows_of(k, b, h, heads, d)[:n], bits, sg, qjl)
                ev = O.tq_write_rows(rows_of(v, b, h, heads, d)[:n], bits, sg, qjl)
                hs = slice(h * group, (h + 1) * group)
                want = O.tq_attention_logits(qq[b, hs], bits, qjl, sg, ek)
                np.testing.assert_allclose(lg[b, hs, :n], want, atol=1e-3, rtol=1e-4)
                ww = w[b, hs, :n]
                want = O.tq_weighted_value_sum(ww, bits, sg, ev)
                vd = np.stack([O.tq_decode(ev[0][t], d, bits, ev[1][t], ev[2][t], sg)
                               for t in range(n)])
                bound = 2.0**-11 * (np.abs(ww) @ np.abs(vd)) + 1e-4 * (1 + np.abs(want))
                assert (np.abs(got[b, hs] - want) <= bound).all(), (b, h)
    finally:
        c.close()


@pytest.mark.parametrize("d,bits,qjl,group,bf16", [(128, 4, True, 4, True), (64, 3, True, 8, False),
                                                    (128, 8, False, 2, False), (256, 4, True, 2, True)])
def test_write_attend_fused_step(rt, d, bits, qjl, group, bf16):
    """sai_tqcache_write_attend against sai_tqcache_write + sai_tqcache_attend
    on a twin cache: the same outputs bit for bit and the same stored rows,
    over ragged lengths (one sequence with several splits, the new row in the
    last), two layers in one pass, two passes."""
    fused_step_case(rt, d, bits, qjl, group, bf16, [2100, 77], 0)


def test_write_attend_fused_step_long_last_split(rt):
    """As above with a 1024-position split: the last split of the first
    sequence holds 14 tiles, more than the workgroup's 8 waves, so the wave
    that stores the new row is the last one, and its own first tile goes to
    the workgroup's tile counter instead. Tiles past a wave's first are
    handed out at run time, so which wave sums which tile can differ between
    any two launches, and each wave rounds its weights to binary16 against
    its own running maximum: the outputs agree to the weights' rounding
    (2^-11 relative; atol 1e-4, rtol 1e-3 here), the stored rows bit for
    bit."""
    prev = rt.set_tq_split(1024)
    try:
        fused_step_case(rt, 128, 4, True, 4, True, [1900, 77], 1024, exact=False)
    finally:
        rt.set_tq_split(prev)


def fused_step_case(rt, d, bits, qjl, group, bf16, lens, split, exact=True):
    import torch
    log(f"tq fused step d={d} bits={bits} qjl={qjl} G={group} bf16={bf16} lens={lens} split={split}")
    rng = np.random.default_rng(group * 3 + bits)
    heads = 2
    batch, nh, cap = len(lens), heads * group, 2200
    twins = [S.TqCache(rt, 2, heads, d, bits, qjl, batch, cap, seed=SEED) for _ in range(2)]
    try:
        k0 = rng.standard_normal((batch, max(lens), heads * d)).astype(np.float32)
        v0 = rng.standard_normal((batch, max(lens), heads * d)).astype(np.float32)
        for c in twins:
            for layer in range(2):
                c.write(layer, to_dev(k0, False), to_dev(v0, False), batch, max(lens))
            c.advance()
            c.set_lengths(lens)
        for step in range(2):
            outs = [[], []]
            for layer in range(2):
                q = to_dev(rng.standard_normal((batch, 1, nh * d)).astype(np.float32), bf16)
                kn = to_dev(rng.standard_normal((batch, 1, heads * d)).astype(np.float32), bf16)
                vn = to_dev(rng.standard_normal((batch, 1, heads * d)).astype(np.float32), bf16)
                for i, c in enumerate(twins):
                    out = torch.zeros((batch, 1, nh * d), device="cuda")
                    if i == 0:
                        c.write(layer, kn, vn, batch, 1)
                        c.attend(layer, q, out, batch, nh)
                    else:
                        c.write_attend(layer, q, kn, vn, out, batch, nh)
                    outs[i].append(out)
            for c in twins:
                c.advance()
            torch.cuda.synchronize()
            for a, b_ in zip(*outs):
                if exact:
                    assert torch.equal(a, b_), step
                else:
                    log(f"  step {step}: max abs diff {(a - b_).abs().max().item():.3e}")
                    assert torch.allclose(a, b_, rtol=1e-3, atol=1e-4), step
        assert list(twins[1].lengths()[0][:batch]) == [n + 2 for n in lens]
        for layer in range(2):
            for b in range(batch):
                for h in range(heads):
                    n = lens[b] + 2
                    r0, r1 = twins[0].read_raw(layer, b, h, n - 3, 3), twins[1].read_raw(layer, b, h, n - 3, 3)
                    for key in r0:
                        assert np.array_equal(r0[key], r1[key]), (layer, b, h, key)
    finally:
        for c in twins:
            c.close()


def test_attend_full_size_sampled(rt):
    """The tq4 workload at full size: 16 sequences x 8192 positions, 32 query
    heads over 8 kv heads, head_dim 128, 4-bit + QJL, bf16 queries; the cache
    filled in 1024-position passes, then the fused write + attend step. The
    outputs of sampled (sequence, kv head) pairs against the oracle, and the
    last stored rows bit for bit."""
    import torch
    log("tq attend full size 16 x 8192, 32Q/8KV, 4-bit + QJL (sampled)")
    batch, heads, group, d, bits, ctx = 16, 8, 4, 128, 4, 8192
    nh = heads * group
    gen = torch.Generator(device="cuda")
    gen.manual_seed(20261202)
    c = S.TqCache(rt, 1, heads, d, bits, True, batch, ctx, seed=SEED)
    try:
        ks, vs = [], []
        for _ in range(ctx // 1024):
            k = torch.randn((batch, 1024, heads * d), generator=gen, device="cuda")
            v = torch.randn((batch, 1024, heads * d), generator=gen, device="cuda")
            c.write(0, k, v, batch, 1024)
            c.advance()
            ks.append(k)
            vs.append(v)
        c.set_lengths([ctx - 1] * batch)
        kn = torch.randn((batch, 1, heads * d), generator=gen, device="cuda").to(torch.bfloat16)
        vn = torch.randn((batch, 1, heads * d), generator=gen, device="cuda").to(torch.bfloat16)
        q = torch.randn((batch, 1, nh * d), generator=gen, device="cuda").to(torch.bfloat16)
        out = torch.zeros((batch, 1, nh * d), device="cuda")
        c.write_attend(0, q, kn, vn, out, batch, nh)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(batch, nh, d)
        k = torch.cat(ks, dim=1)[:, :ctx - 1].float().cpu().numpy()
        v = torch.cat(vs, dim=1)[:, :ctx - 1].float().cpu().numpy()
        k = np.concatenate([k, kn.float().cpu().numpy()], axis=1)
        v = np.concatenate([v, vn.float().cpu().numpy()], axis=1)
        qq = q.float().cpu().numpy().reshape(batch, nh, d)
        for b, h in [(0, 0), (7, 5), (15, 7)]:
            sg = head_signs(SEED, 0, heads, h, d)
            want = oracle_attend(rows_of(k, b, h, heads, d), rows_of(v, b, h, heads, d),
                                 qq[b, h * group:(h + 1) * group], bits, True, sg,
                                 S.default_scale(d))
            np.testing.assert_allclose(got[b, h * group:(h + 1) * group], want, atol=2e-3,
                                       rtol=1e-2)
            check_rows(c, 0, b, h, ctx - 4, rows_of(k, b, h, heads, d)[ctx - 4:],
                       rows_of(v, b, h, heads, d)[ctx - 4:], heads, d, bits, True, SEED)
    finally:
        c.close()


def test_empty_sequence_gives_zero_rows(rt):
    """A sequence with no rows in the batch (set_lengths 0, nothing pending):
    attention and the weighted sum write zero rows for it, as the reference's
    SDPA does for a row with no visible key; the other sequence is unaffected."""
    import torch
    d, heads, group = 128, 2, 4
    nh = heads * group
    c = S.TqCache(rt, 1, heads, d, 4, True, 2, 64, seed=SEED)
    try:
        x = torch.randn(2, 10, heads * d, device="cuda")
        c.write(0, x, x, 2, 10)
        c.advance()
        c.set_lengths([10, 0])
        q = torch.randn(2, 1, nh * d, device="cuda")
        out = torch.full((2, 1, nh * d), float("nan"), device="cuda")
        c.attend(0, q, out, 2, nh)
        w = torch.ones(2 * nh, 16, device="cuda")
        ws = torch.full((2, 1, nh * d), float("nan"), device="cuda")
        c.weighted_value_sum(0, w, 16, ws, 2, nh)
        torch.cuda.synchronize()
        assert torch.equal(out[1], torch.zeros_like(out[1]))
        assert torch.equal(ws[1], torch.zeros_like(ws[1]))
        assert torch.isfinite(out[0]).all() and torch.isfinite(ws[0]).all()
    finally:
        c.close()


def test_memory_bytes(rt):
    """cache_memory_footprint (kv_compression.rs:1517-1547): 128 rows of D=64,
    4-bit + QJL stay below the f32 size; the count follows the reference's
    per-block (packed + 25 B) and per-residual (words * 8 + 12 B) sizes."""
    import torch
    d = 64
    c = S.TqCache(rt, 1, 1, d, 4, True, 1, 128, seed=42)
    try:
        pos = np.arange(128, dtype=np.float32)[:, None]
        k = ((np.arange(d, dtype=np.float32)[None] + pos) * np.float32(0.01)).reshape(1, 128, d)
        v = ((np.arange(d, dtype=np.float32)[None] + pos + 100) * np.float32(0.01)).reshape(1, 128, d)
        assert c.memory_bytes()[0] == 0
        c.write(0, to_dev(k.astype(np.float32), False), to_dev(v.astype(np.float32), False), 1, 128)
        c.advance()
        torch.cuda.synchronize()
        ref, dev = c.memory_bytes()
        assert ref < 128 * d * 4 * 2
        assert ref == 128 * (2 * (32 + 25) + 2 * (8 + 12))
        assert dev >= 128 * (2 * 32 + 32)
    finally:
        c.close()


def test_errors_and_lifecycle(rt):
    import torch
    with pytest.raises(S.SaiError) as e:
        S.TqCache(rt, 1, 2, 64, 5, True, 1, 8)
    assert e.value.kind == "InvalidAttribute" and "bits must be 3, 4, or 8" in str(e.value)
    with pytest.raises(S.SaiError) as e:
        S.TqCache(rt, 1, 2, 96, 4, True, 1, 8)
    assert e.value.kind == "Unsupported"
    c256 = S.TqCache(rt, 1, 1, 256, 4, True, 1, 8)
    try:
        import torch
        x = torch.randn(1, 1, 256, device="cuda")
        c256.write(0, x, x, 1, 1)
        with pytest.raises(S.SaiError) as e:  # group 8 at head_dim 256
            c256.attend(0, torch.randn(1, 1, 8 * 256, device="cuda"),
                        torch.zeros(1, 1, 8 * 256, device="cuda"), 1, 8)
        assert e.value.kind == "Unsupported"
    finally:
        c256.close()
    d, heads = 64, 2
    c = S.TqCache(rt, 2, heads, d, 4, False, 2, 8)
    try:
        x = torch.randn(2, 6, heads * d, device="cuda")
        c.write(0, x, x, 2, 6)
        with pytest.raises(S.SaiError) as e:  # the pass appends 6 rows
            c.write(1, x[:, :1], x[:, :1], 2, 1)
        assert e.value.kind == "ShapeMismatch"
        c.advance()
        with pytest.raises(S.SaiError) as e:  # 6 + 6 > 8
            c.write(0, x, x, 2, 6)
        assert e.value.kind == "PositionOverflow"
        with pytest.raises(S.SaiError) as e:
            c.write(2, x, x, 2, 1)
        assert e.value.kind == "ShapeMismatch"
        q = torch.randn(2, 1, 3 * d, device="cuda")
        out = torch.zeros(2, 1, 3 * d, device="cuda")
        with pytest.raises(S.SaiError) as e:  # 3 query heads over 2 kv heads
            c.attend(0, q, out, 2, 3)
        assert e.value.kind == "InvalidAttribute"
        with pytest.raises(S.SaiError) as e:
            c.read(0, 0, 0, 4, 3)
        assert e.value.kind == "ShapeMismatch"
        c.reset()
        lens, pend, _ = c.lengths()
        assert not lens.any() and pend == 0
        with pytest.raises(S.SaiError) as e:
            c.attend(0, q[:, :, :2 * d].contiguous(), out, 2, 2)
        assert e.value.kind == "ShapeMismatch"
    finally:
        c.close()


def test_attend_reproducible_tile_order(rt):
    """sai_set_decode_reproducible(1) fixes the attention's tile order too:
    repeated calls over one cache (1024-position splits of 16 tiles over 8
    waves, so most tiles are past the waves' first) give bit-identical
    outputs; the default run-time order stays within the weights' rounding
    of them."""
    import torch
    log("tq attend: fixed tile order, repeated calls")
    rng = np.random.default_rng(0x7A11)
    d, bits, qjl, group, heads = 128, 4, True, 4, 2
    lens = [1900, 1500, 77]
    batch, nh = len(lens), heads * group
    c = S.TqCache(rt, 1, heads, d, bits, qjl, batch, 2048, seed=SEED)
    prev_s = rt.set_tq_split(1024)
    prev_r = rt.set_decode_reproducible(1)
    try:
        k0 = rng.standard_normal((batch, max(lens), heads * d)).astype(np.float32)
        v0 = rng.standard_normal((batch, max(lens), heads * d)).astype(np.float32)
        c.write(0, to_dev(k0, False), to_dev(v0, False), batch, max(lens))
        c.advance()
        c.set_lengths(lens)
        q = to_dev(rng.standard_normal((batch, 1, nh * d)).astype(np.float32), True)
        outs = []
        for mode in (1, 1, 1, 0):
            rt.set_decode_reproducible(mode)
            out = torch.zeros((batch, 1, nh * d), device="cuda")
            c.attend(0, q, out, batch, nh)
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
        diff = (outs[3] - outs[0]).abs().max().item()
        log(f"  run-time vs fixed order: max abs diff {diff:.3e}")
        assert torch.allclose(outs[3], outs[0], rtol=1e-3, atol=1e-4)
    finally:
        rt.set_decode_reproducible(prev_r)
        rt.set_tq_split(prev_s)
        c.close()


def test_attend_split_merge_handoff_repeated(rt):
    """The attention's in-kernel split merge (agent-scope partial stores, their
    completion, the ticket, the last holder's loads) over many splits: with the
    smallest split, 256 positions, three sequences make up to 8 splits each, and 30
    calls with the fixed tile order give the same bits every time (a partial read
    before its store landed would change an output)."""
    import torch
    log("tq attend: split merge handoff, 256-position splits, 30 calls")
    rng = np.random.default_rng(0x7A12)
    d, bits, qjl, group, heads = 128, 4, True, 4, 2
    lens = [1900, 1500, 77]
    batch, nh = len(lens), heads * group
    c = S.TqCache(rt, 1, heads, d, bits, qjl, batch, 2048, seed=SEED)
    prev_s = rt.set_tq_split(256)
    prev_r = rt.set_decode_reproducible(1)
    try:
        k0 = rng.standard_normal((batch, max(lens), heads * d)).astype(np.float32)
        v0 = rng.standard_normal((batch, max(lens), heads * d)).astype(np.float32)
        c.write(0, to_dev(k0, False), to_dev(v0, False), batch, max(lens))
        c.advance()
        c.set_lengths(lens)
        q = to_dev(rng.standard_normal((batch, 1, nh * d)).astype(np.float32), True)
        outs = []
        for _ in range(30):
            out = torch.zeros((batch, 1, nh * d), device="cuda")
            c.attend(0, q, out, batch, nh)
            outs.append(out)
        torch.cuda.synchronize()
        for i, o in enumerate(outs[1:], 1):
            assert torch.equal(o, outs[0]), f"call {i} differs"
        assert torch.isfinite(outs[0]).all()
    finally:
        rt.set_decode_reproducible(prev_r)
        rt.set_tq_split(prev_s)
        c.close()
