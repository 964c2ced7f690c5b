"""A seeded random sweep of the decode, fused-step, prefill and TurboQuant
decode paths over the supported shapes and options, every case against the
oracle through the C ABI.

The targeted tests pin one option at a time; this sweep draws them together
(quantisation, head_dim 64/128/168/256, GQA group 1-8, ragged lengths from 0
to a few thousand, f32/bf16 K/V, query and output, RoPE on/off and its pair
layout, permuted pages, forced split sizes, the three merge modes, the two
tile orders, node and layer windows), so that combinations no single test
names still meet the bar: outputs within 2e-3 abs + 1e-2 rel of the oracle
(bf16 outputs: that bar widened by bf16's rounding), and the stored codes
bit-exact where a case checks them. The TurboQuant cases draw head_dim, bits,
QJL, group, lengths, bf16 inputs, the split, the tile order, the scale and the
fused or separate store, against the oracle's encode and attention at the same
bar; the append cases, three appends of random sizes after a random past, keep
every code and scale bit-exact. Each case prints its draw before it runs.
"""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import Case, assert_close, bf16_tol_close, log, to_bf16_f32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    assert S.lib().sai_device_supported(0) == 1, "device 0 is not gfx950"
    r = S.Runtime(0)
    yield r
    r.close()


def _pick(rng, xs):
    return xs[int(rng.integers(0, len(xs)))]


def _shape(rng, max_rows):
    """quant, head_dim, kv heads, query heads (the supported combinations)."""
    quant = _pick(rng, [S.KV_INT8, S.KV_INT4])
    d = _pick(rng, [64, 128, 168, 256] if quant == S.KV_INT8 else [64, 128, 256])
    groups = [1, 2, 4] if (quant == S.KV_INT4 and d == 256) else [1, 2, 4, 8]
    g = _pick(rng, groups)
    hkv = _pick(rng, [1, 2, 3, 4])
    # keep the oracle's work to about a second per case
    while hkv > 1 and hkv * g * d * max_rows > 24_000_000:
        hkv -= 1
    return quant, d, hkv, hkv * g


def _draw_decode(i):
    rng = np.random.default_rng(0x5EE90000 + i)
    batch = int(rng.integers(1, 5))
    max_len = _pick(rng, [64, 700, 3000])
    lens = [int(x) for x in rng.integers(0, max_len, batch)]
    quant, d, hkv, hq = _shape(rng, batch * max_len)
    return dict(
        seed=0x5EE90000 + i, quant=quant, d=d, hkv=hkv, hq=hq, lens=lens,
        kv_dtype=_pick(rng, ["f32", "bf16"]), q_dtype=_pick(rng, ["f32", "bf16"]),
        out_dtype=_pick(rng, ["f32", "f32", "bf16"]),
        rotary=bool(rng.random() < 0.8), interleaved=bool(rng.random() < 0.3),
        permute=bool(rng.random() < 0.5), fused=bool(rng.random() < 0.5),
        split=_pick(rng, [0, 0, 64, 192, 512, 1024, 2048]), merge=_pick(rng, [0, 1, 2]),
        reproducible=_pick(rng, [0, 1, 2]),
        window=_pick(rng, [0, 0, 0, 1, 37, 500]),
        layer_window=_pick(rng, [0, 0, 0, 64, 300]),
        theta=_pick(rng, [1e4, 5e5]))


def _draw_prefill(i):
    rng = np.random.default_rng(0x9EF10000 + i)
    batch = int(rng.integers(1, 4))
    past = [int(x) for x in rng.integers(0, _pick(rng, [1, 200, 1500, 6000]), batch)]
    new = int(_pick(rng, [1, 5, 64, 130, 300]))
    quant, d, hkv, hq = _shape(rng, batch * (max(past) + new) * 4)
    return dict(
        seed=0x9EF10000 + i, quant=quant, d=d, hkv=hkv, hq=hq, past=past, new=new,
        kv_dtype=_pick(rng, ["f32", "bf16"]), q_dtype=_pick(rng, ["f32", "bf16"]),
        out_dtype=_pick(rng, ["f32", "f32", "bf16"]),
        rotary=bool(rng.random() < 0.8), interleaved=bool(rng.random() < 0.3),
        permute=bool(rng.random() < 0.5),
        window=_pick(rng, [0, 0, 0, 1, 50, 400]),
        layer_window=_pick(rng, [0, 0, 0, 33, 256]),
        theta=_pick(rng, [1e4, 5e5]))


def _check(got, ref, out_dtype, what):
    if out_dtype == "bf16":
        bf16_tol_close(got, ref, what)
    else:
        assert_close(got, ref, what)


@pytest.mark.parametrize("i", range(96))
def test_decode_sweep(rt, i):
    cfg = _draw_decode(i)
    log(f"decode sweep {i}: {cfg}")
    prev_split = rt.set_decode_split(cfg["split"])
    prev_merge = rt.set_decode_merge(cfg["merge"])
    prev_rep = rt.set_decode_reproducible(cfg["reproducible"])
    try:
        fused = cfg["fused"]
        c = Case(rt, cfg["seed"], len(cfg["lens"]), cfg["hq"], cfg["hkv"], cfg["d"], cfg["lens"],
                 0 if fused else 1, theta=cfg["theta"], quant=cfg["quant"],
                 kv_dtype=cfg["kv_dtype"], permute_pages=cfg["permute"],
                 do_rotary=cfg["rotary"], interleaved=cfg["interleaved"],
                 extra_tokens=1 if fused else 0)
        c.cache.set_layer_window(0, cfg["layer_window"])
        q = c.rng.standard_normal((c.batch, 1, c.hq * c.d), dtype=np.float32)
        if cfg["q_dtype"] == "bf16":
            q = to_bf16_f32(q)
        if fused:
            got = c.step_fused(q, cfg["q_dtype"], window=cfg["window"], out_dtype=cfg["out_dtype"])
        else:
            c.step_kv()
            got = c.gpu_decode(q, cfg["q_dtype"], window=cfg["window"],
                               out_dtype=cfg["out_dtype"])
        ref = c.oracle_attend(q, layer_window=cfg["layer_window"], mask_window=cfg["window"])
        _check(got, ref, cfg["out_dtype"], f"decode sweep {i}")
        if fused:
            c.check_codes()
    finally:
        rt.set_decode_split(prev_split)
        rt.set_decode_merge(prev_merge)
        rt.set_decode_reproducible(prev_rep)


@pytest.mark.parametrize("i", range(96))
def test_prefill_sweep(rt, i):
    cfg = _draw_prefill(i)
    log(f"prefill sweep {i}: {cfg}")
    c = Case(rt, cfg["seed"], len(cfg["past"]), cfg["hq"], cfg["hkv"], cfg["d"], cfg["past"],
             cfg["new"], theta=cfg["theta"], quant=cfg["quant"], kv_dtype=cfg["kv_dtype"],
             permute_pages=cfg["permute"], do_rotary=cfg["rotary"],
             interleaved=cfg["interleaved"])
    c.cache.set_layer_window(0, cfg["layer_window"])
    c.step_kv()
    q = c.query(cfg["q_dtype"])
    got = c.gpu_prefill(q, cfg["q_dtype"], window=cfg["window"], out_dtype=cfg["out_dtype"])
    ref = c.oracle_attend(q, layer_window=cfg["layer_window"], mask_window=cfg["window"])
    _check(got, ref, cfg["out_dtype"], f"prefill sweep {i}")
    c.check_codes(seqs=[0])


TQ_SEED = 0x7A5E


def _draw_tq(i):
    rng = np.random.default_rng(0x79000000 + i)
    d = _pick(rng, [64, 128, 256])
    return dict(
        d=d, bits=_pick(rng, [3, 4, 8]), qjl=bool(rng.random() < 0.6),
        group=_pick(rng, [1, 2, 4] if d == 256 else [1, 2, 4, 8]),
        heads=int(rng.integers(1, 4)), lens=[int(x) for x in rng.integers(
            0, _pick(rng, [70, 900, 2500]), int(rng.integers(1, 4)))],
        bf16=bool(rng.random() < 0.4), fused=bool(rng.random() < 0.5),
        split=_pick(rng, [0, 0, 256, 512, 1024]), reproducible=_pick(rng, [0, 1, 2]),
        scale=_pick(rng, [None, None, 0.05]))


@pytest.mark.parametrize("i", range(48))
def test_turboquant_attend_sweep(rt, i):
    """The TurboQuant decode step (a pending row stored by the write kernel or
    by the fused write_attend, then attended) against the oracle's encode and
    attention, per (sequence, kv head)."""
    import torch
    from test_gpu_turboquant import head_signs, host_vals, oracle_attend, rows_of, to_dev
    cfg = _draw_tq(i)
    log(f"turboquant sweep {i}: {cfg}")
    d, bits, qjl, group, heads = cfg["d"], cfg["bits"], cfg["qjl"], cfg["group"], cfg["heads"]
    lens, bf16 = cfg["lens"], cfg["bf16"]
    batch, nh, rows = len(lens), heads * cfg["group"], max(lens)
    rng = np.random.default_rng(0x79100000 + i)
    prev_split = rt.set_tq_split(cfg["split"])
    prev_rep = rt.set_decode_reproducible(cfg["reproducible"])
    c = S.TqCache(rt, 1, heads, d, bits, qjl, batch, rows + 1, seed=TQ_SEED)
    try:
        k0 = rng.standard_normal((batch, max(rows, 1), heads * d)).astype(np.float32)
        v0 = rng.standard_normal((batch, max(rows, 1), heads * d)).astype(np.float32)
        if rows > 0:
            c.write(0, to_dev(k0, bf16), to_dev(v0, bf16), batch, rows)
            c.advance()
            c.set_lengths(lens)
        kn = rng.standard_normal((batch, 1, heads * d)).astype(np.float32)
        vn = rng.standard_normal((batch, 1, heads * d)).astype(np.float32)
        q = rng.standard_normal((batch, 1, nh * d)).astype(np.float32)
        out = torch.full((batch, 1, nh * d), float("nan"), device="cuda")
        if cfg["fused"]:
            c.write_attend(0, to_dev(q, bf16), to_dev(kn, bf16), to_dev(vn, bf16), out, batch, nh,
                           scale=cfg["scale"])
        else:
            c.write(0, to_dev(kn, bf16), to_dev(vn, bf16), batch, 1)
            c.attend(0, to_dev(q, bf16), out, batch, nh, scale=cfg["scale"])
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(batch, nh, d)
        kk, vv = host_vals(k0, bf16), host_vals(v0, bf16)
        kn_h, vn_h = host_vals(kn, bf16), host_vals(vn, bf16)
        qq = host_vals(q, bf16).reshape(batch, nh, d)
        scale = S.default_scale(d) if cfg["scale"] is None else cfg["scale"]
        for b in range(batch):
            n = lens[b]
            for h in range(heads):
                sg = head_signs(TQ_SEED, 0, heads, h, d)
                rk = np.concatenate([rows_of(kk, b, h, heads, d)[:n], rows_of(kn_h, b, h, heads, d)])
                rv = np.concatenate([rows_of(vv, b, h, heads, d)[:n], rows_of(vn_h, b, h, heads, d)])
                want = oracle_attend(rk, rv, qq[b, h * group:(h + 1) * group], bits, qjl, sg, scale)
                np.testing.assert_allclose(got[b, h * group:(h + 1) * group], want, atol=2e-3,
                                           rtol=1e-2, err_msg=f"sweep {i} b={b} h={h}")
    finally:
        c.close()
        rt.set_tq_split(prev_split)
        rt.set_decode_reproducible(prev_rep)


def _draw_append(i):
    rng = np.random.default_rng(0xA99E0000 + i)
    batch = int(rng.integers(1, 5))
    quant, d, hkv, _ = _shape(rng, 1)
    return dict(
        seed=0xA99E0000 + i, quant=quant, d=d, hkv=hkv,
        past=[int(x) for x in rng.integers(0, _pick(rng, [1, 20, 300]), batch)],
        steps=[int(_pick(rng, [1, 2, 3, 4, 7, 16, 17, 40, 100])) for _ in range(3)],
        kv_dtype=_pick(rng, ["f32", "bf16"]), rotary=bool(rng.random() < 0.8),
        interleaved=bool(rng.random() < 0.3), permute=bool(rng.random() < 0.5),
        theta=_pick(rng, [1e4, 5e5]))


@pytest.mark.parametrize("i", range(48))
def test_append_sweep(rt, i):
    """Three appends of random sizes (the row kernel below 4 tokens, the page
    kernel from 4, partial first and last pages) after a random committed
    past; every stored code and scale bit-exact against the oracle."""
    cfg = _draw_append(i)
    log(f"append sweep {i}: {cfg}")
    total = sum(cfg["steps"])
    c = Case(rt, cfg["seed"], len(cfg["past"]), cfg["hkv"], cfg["hkv"], cfg["d"], cfg["past"],
             0, theta=cfg["theta"], quant=cfg["quant"], kv_dtype=cfg["kv_dtype"],
             permute_pages=cfg["permute"], do_rotary=cfg["rotary"],
             interleaved=cfg["interleaved"], extra_tokens=total)
    for n in cfg["steps"]:
        k, v = c.kv(n)
        c.append_both(k, v)
        c.cache.advance()
    c.check_codes()


def _draw_wide(i):
    """int8 at head_dim 168 and 256: the decode's single phased tile buffer,
    with several tiles per wave (long sequences, large splits)."""
    rng = np.random.default_rng(0x5A560000 + i)
    batch = int(rng.integers(1, 4))
    d = _pick(rng, [168, 256])
    g = _pick(rng, [1, 2, 4, 8])
    return dict(
        seed=0x5A560000 + i, quant=S.KV_INT8, d=d, hkv=_pick(rng, [1, 2]), g=g,
        lens=[int(x) for x in rng.integers(0, 6000, batch)],
        kv_dtype=_pick(rng, ["f32", "bf16"]), q_dtype=_pick(rng, ["f32", "bf16"]),
        out_dtype=_pick(rng, ["f32", "bf16"]), rotary=bool(rng.random() < 0.8),
        interleaved=bool(rng.random() < 0.3), permute=bool(rng.random() < 0.5),
        fused=bool(rng.random() < 0.5), split=_pick(rng, [0, 512, 1024, 2048, 4096]),
        merge=_pick(rng, [0, 1, 2]), reproducible=_pick(rng, [0, 1, 2]),
        window=_pick(rng, [0, 0, 700]), layer_window=_pick(rng, [0, 0, 1024]),
        theta=1e6)


@pytest.mark.parametrize("i", range(32))
def test_decode_wide_heads_sweep(rt, i):
    cfg = _draw_wide(i)
    cfg = dict(cfg, hq=cfg["hkv"] * cfg["g"])
    log(f"wide-head decode sweep {i}: {cfg}")
    prev_split = rt.set_decode_split(cfg["split"])
    prev_merge = rt.set_decode_merge(cfg["merge"])
    prev_rep = rt.set_decode_reproducible(cfg["reproducible"])
    try:
        fused = cfg["fused"]
        c = Case(rt, cfg["seed"], len(cfg["lens"]), cfg["hq"], cfg["hkv"], cfg["d"], cfg["lens"],
                 0 if fused else 1, theta=cfg["theta"], quant=cfg["quant"],
                 kv_dtype=cfg["kv_dtype"], permute_pages=cfg["permute"],
                 do_rotary=cfg["rotary"], interleaved=cfg["interleaved"],
                 extra_tokens=1 if fused else 0)
        c.cache.set_layer_window(0, cfg["layer_window"])
        q = c.rng.standard_normal((c.batch, 1, c.hq * c.d), dtype=np.float32)
        if cfg["q_dtype"] == "bf16":
            q = to_bf16_f32(q)
        if fused:
            got = c.step_fused(q, cfg["q_dtype"], window=cfg["window"], out_dtype=cfg["out_dtype"])
        else:
            c.step_kv()
            got = c.gpu_decode(q, cfg["q_dtype"], window=cfg["window"],
                               out_dtype=cfg["out_dtype"])
        ref = c.oracle_attend(q, layer_window=cfg["layer_window"], mask_window=cfg["window"])
        _check(got, ref, cfg["out_dtype"], f"wide-head decode sweep {i}")
    finally:
        rt.set_decode_split(prev_split)
        rt.set_decode_merge(prev_merge)
        rt.set_decode_reproducible(prev_rep)
