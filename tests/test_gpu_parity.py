"""GPU parity of the three HIP kernels against the CPU oracle, through the C ABI.

Bar: KV codes and scales bit-exact; attention outputs within 2e-3 abs + 1e-2 rel
of the oracle (the reference's f32 CPU semantics over the dequantised cache).
Shapes follow the five workloads of the path (decode batch 1 / Llama-3-8B layer
/ int4 long context / ragged paged batch / prefill chunk), at full size where
the oracle finishes in seconds and at reduced length otherwise.
"""
import numpy as np
import pytest

import smallaios_amd as S
from _gpu_util import (Case, assert_close, assert_close_weighted, dev, err_tol_ratio, log,
                       outlier_student_t, weighted_abs_v)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    assert S.lib().sai_device_supported(0) == 1, "device 0 is not gfx950"
    r = S.Runtime(0)
    yield r
    r.close()


# ----------------------------------------------------------------- append ---
def test_append_c1_int8_bit_exact(rt):
    log("append c1: B=1 Hkv=2 D=64 past=511 +1, f32, theta 1e4")
    c = Case(rt, 0x5A1A0000, 1, 8, 2, 64, [511], 1, theta=1e4)
    c.step_kv()
    c.check_codes()


@pytest.mark.parametrize("d,interleaved,rot,kv_dtype", [
    (128, False, True, "bf16"), (128, True, True, "f32"), (64, True, True, "f32"),
    (128, False, False, "f32")])
def test_append_variants_bit_exact(rt, d, interleaved, rot, kv_dtype):
    log(f"append variants d={d} interleaved={interleaved} rotary={rot} {kv_dtype}")
    c = Case(rt, 7 + d, 3, 8, 4, d, [40, 5, 17], 9, theta=5e5, kv_dtype=kv_dtype,
             permute_pages=True, interleaved=interleaved, do_rotary=rot)
    c.step_kv()
    c.check_codes()


@pytest.mark.parametrize("hkv", [2, 3, 8])
@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
@pytest.mark.parametrize("d,interleaved,kv_dtype", [
    (64, False, "f32"), (64, True, "bf16"), (128, False, "bf16"), (128, True, "f32"),
    (256, False, "bf16"), (256, True, "f32")])
def test_append_page_blocks_bit_exact(rt, d, interleaved, kv_dtype, quant, hkv):
    """Multi-token appends take the page-block kernel (one workgroup per page
    block, 16-byte stores): 20 new tokens from starts 13, 0, 31 and 16 span
    two or three pages, first and last page partial or whole; the slots
    before the start keep their codes (int4: the other nibble of each V
    byte). 3 tokens take the per-row (int4: per-pair) kernel, and the results
    of both meet bit-exact in one cache. K with x20 outlier channels and
    heavy tails, so the int4 groups' ranges differ widely. 2, 3 and 8 kv
    heads: the int4 form puts 1 to 8 kv heads in one workgroup."""
    log(f"append page blocks quant={quant} d={d} hkv={hkv} interleaved={interleaved} {kv_dtype}")
    from _gpu_util import outlier_keys
    c = Case(rt, 0xB10C + d + hkv, 4, 8, hkv, d, [13, 0, 31, 16], 20, theta=5e5,
             kv_dtype=kv_dtype, permute_pages=True, interleaved=interleaved, extra_tokens=3, quant=quant,
             k_transform=outlier_keys(d, channels=(5, 17, d - 3)))
    c.step_kv()
    c.check_codes()
    c.cache.advance()
    k, v = c.kv(3)
    c.append_both(k, v)
    c.check_codes()


def test_append_unaligned_rows_bit_exact(rt):
    """Rows that do not start 16-byte aligned (a view 4 bytes into its
    buffer) are appended by the per-row kernel, with the same codes."""
    import torch
    log("append: 4-byte-offset K/V views, 12 tokens")
    c = Case(rt, 0xA11, 2, 8, 2, 128, [5, 22], 12, theta=5e5, permute_pages=True)
    k, v = c.kv(12)

    def offset_view(x):
        flat = torch.zeros(x.size + 1, dtype=torch.float32, device="cuda")
        flat[1:] = torch.from_numpy(x.reshape(-1)).cuda()
        view = flat[1:].view(x.shape)
        assert view.data_ptr() % 16 == 4
        return view

    kd, vd = offset_view(k), offset_view(v)
    c.cache.append(0, kd, vd, c.batch, 12, c.cos_d, c.sin_d, c.cos.shape[0], True, False)
    c.ocache.append(k, v, c.cos, c.sin, True, False)
    torch.cuda.synchronize()
    c.check_codes()


@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
def test_append_special_values(rt, quant):
    """Zero rows, huge/tiny magnitudes, inf and NaN keep the codes (and int4's
    binary16 group parameters) bit-exact; 8 tokens take the page-block
    kernel."""
    log(f"append special values quant={quant}")

    def poison(rng, k):
        k = k.copy()
        k[0, 0, :64] = 0.0                      # zero row -> scale 1.0
        k[0, 1, :64] = np.float32(3.0e38)       # huge
        k[0, 2, :64] *= np.float32(1e-30)       # tiny
        k[0, 3, 5] = np.inf
        k[0, 4, 7] = np.nan
        k[0, 5, :64] = np.nan                   # all-NaN row
        k[0, 6, 64:128] = np.float32(-np.inf)
        return k

    c = Case(rt, 11, 1, 4, 2, 64, [0], 8, k_transform=poison, do_rotary=False, quant=quant)
    c.step_kv()
    c.check_codes()


def signed_zero_groups(rng, x):
    """Positive values with groups of 32 whose minimum is zero: +0 before -0 and the
    reverse, in one lane of the page kernel (dims 4k .. 4k+3) and in different lanes, a
    lone -0, an all-zero group of mixed signs, and zeros beside a negative minimum."""
    b, n, hd = x.shape
    x = (np.abs(x) + np.float32(0.25)).reshape(b, n, hd // 32, 32).copy()
    pz, nz = np.float32(0.0), np.float32(-0.0)
    for t in range(n):
        for g in range(hd // 32):
            p = (t + 3 * g) % 7
            row = x[:, t, g]
            if p == 0:
                row[:, 3], row[:, 10] = pz, nz
            elif p == 1:
                row[:, 2], row[:, 20] = nz, pz
            elif p == 2:
                row[:, 31] = nz
            elif p == 3:
                row[:, 7], row[:, 5] = nz, pz
            elif p == 4:
                row[:, 6], row[:, 4] = pz, nz
            elif p == 5:
                row[:] = np.where(np.arange(32) % 2 == 0, nz, pz)
            else:
                row[:, 0], row[:, 1], row[:, 9] = pz, nz, np.float32(-1.0)
    return x.reshape(b, n, hd)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_append_int4_signed_zero_minimum(rt, d, kv_dtype):
    """A group whose minimum is zero stores the sign of its first zero in dim order as its
    binary16 zero point: the reference's scan keeps the first of equal minima
    (kv_compression.rs:227-235). Through the page kernel (30 tokens), the per-pair kernel
    (3 tokens) and the fused decode step."""
    log(f"append int4 signed-zero minima d={d} {kv_dtype}")
    c = Case(rt, 0x5E20 + d, 2, 8, 2, d, [13, 30], 1, quant=S.KV_INT4, kv_dtype=kv_dtype,
             do_rotary=False, permute_pages=True, extra_tokens=4,
             k_transform=signed_zero_groups, v_transform=signed_zero_groups)
    c.check_codes()
    k, v = c.kv(3)
    c.append_both(k, v)
    c.check_codes()
    c.cache.advance()
    q = c.query()
    got = c.step_fused(q)
    assert_close(got, c.oracle_attend(q), "fused step after signed-zero groups")
    c.check_codes()


def test_append_int4_bit_exact(rt):
    """int4 asym g32 codes and f16 params, K with x20 outlier channels."""
    log("append int4: outlier channels, student-t, odd start positions")

    c = Case(rt, 0x5A1A0002, 2, 8, 2, 128, [33, 6], 5, theta=5e5, quant=S.KV_INT4,
             k_transform=outlier_student_t, permute_pages=True, extra_tokens=1)
    c.step_kv()
    c.check_codes()
    c.cache.advance()
    # a single-token append at an odd position must keep the neighbour's nibble
    k, v = c.kv(1)
    c.append_both(k, v)
    c.check_codes()


# ----------------------------------------------------------------- decode ---
def test_decode_c1(rt):
    log("decode c1: 8Q/2KV D=64 ctx 512 B=1 f32 theta 1e4")
    c = Case(rt, 0x5A1A0000, 1, 8, 2, 64, [511], 1, theta=1e4)
    c.step_kv()
    q = c.query()
    got = c.gpu_decode(q)
    ref = c.oracle_attend(q)
    err = assert_close(got, ref, "c1 decode")
    log(f"  max abs err {err:.2e}")


def test_decode_llama_shape_ragged_bf16(rt):
    log("decode 32Q/8KV D=128 B=4 ragged, bf16, permuted pages, theta 5e5")
    c = Case(rt, 21, 4, 32, 8, 128, [1000, 77, 513, 2047], 1, theta=5e5, kv_dtype="bf16",
             permute_pages=True)
    c.step_kv()
    q = c.query("bf16")
    got = c.gpu_decode(q, "bf16")
    ref = c.oracle_attend(q)
    assert_close(got, ref, "llama-shape decode")
    c.check_codes(seqs=[1])


@pytest.mark.parametrize("hq,hkv,d", [(4, 4, 128), (8, 4, 64), (32, 4, 128), (16, 2, 64)])
def test_decode_groups(rt, hq, hkv, d):
    log(f"decode group {hq // hkv}: hq={hq} hkv={hkv} d={d}")
    c = Case(rt, 31 + hq, 2, hq, hkv, d, [300, 129], 1, permute_pages=True)
    c.step_kv()
    q = c.query()
    assert_close(c.gpu_decode(q), c.oracle_attend(q), f"group {hq // hkv}")


@pytest.mark.parametrize("split", [64, 256, 1024])
def test_decode_split_merge(rt, split):
    """Many split-K partials merged by the last workgroup; repeated launches
    reuse the self-resetting counters."""
    log(f"decode split merge split={split}")
    c = Case(rt, 41, 3, 32, 8, 128, [3000, 1, 640], 1, permute_pages=True)
    prev = rt.set_decode_split(split)
    try:
        c.step_kv()
        q = c.query()
        ref = c.oracle_attend(q)
        for _ in range(3):
            assert_close(c.gpu_decode(q), ref, f"split {split}")
        wg, sp = rt.last_decode_shape()
        assert sp == split and wg >= 8
    finally:
        rt.set_decode_split(prev)


@pytest.mark.parametrize("merge", [0, 1, 2])
@pytest.mark.parametrize("split", [64, 4096])
def test_decode_fused_step(rt, merge, split):
    """sai_gqa_with_cache: the decode kernel appends the token itself (codes
    bit-exact with the standalone append) and merges splits in the combine
    kernel (0), in-kernel (1) or as chosen automatically (2); repeated steps
    advance the cache."""
    log(f"fused decode step merge={merge} split={split}")
    prev_m = rt.set_decode_merge(merge)
    prev_s = rt.set_decode_split(split)
    try:
        c = Case(rt, 91, 3, 32, 8, 128, [700, 5, 4100], 1, theta=5e5, kv_dtype="bf16",
                 permute_pages=True, extra_tokens=2)
        for step in range(3):
            q = c.query("bf16")
            got = c.step_fused(q, "bf16")
            assert_close(got, c.oracle_attend(q), f"fused step {step}")
            c.check_codes(seqs=[1])
            c.cache.advance()
    finally:
        rt.set_decode_merge(prev_m)
        rt.set_decode_split(prev_s)


@pytest.mark.parametrize("quant,vscale", [
    (S.KV_INT8, 1.0e5), (S.KV_INT8, 1.0e7), (S.KV_INT4, 1.0e4),
])
@pytest.mark.parametrize("split", [256, 0])
def test_decode_large_v(rt, quant, vscale, split):
    """The fused decode step (sai_gqa_with_cache) with V rows of |v| ~ 4e5 or
    4e7 and keys at 300-339 scaled x6 (weights concentrated on a few keys
    whose V rows cancel far below |v|), one split and many. int8 P' is two
    int8 terms against its 64-token tile's maximum, int4 P' one binary16
    value per (head, group); both are scale-free, so the outputs are checked
    against the bound of that representation (decode_weight_bounds) plus the
    oracle's expf_approx error, on top of 2e-3 + 1e-2|ref| (the oracle's
    expf_approx alone moves such outputs by more than 2e-3). int4 runs at
    1e4 (|v| ~ 4e4): its zero point, the group minimum, is stored as
    binary16, so V beyond 65504 is outside the scheme (inf in the oracle
    too)."""
    from _gpu_util import assert_close_decode_bound, decode_weight_bounds
    log(f"decode large V: quant {quant} V x{vscale:g} split {split}")

    def jump(rng, k):
        if k.shape[1] >= 340:
            k[:, 300:340] *= 6.0
        return k

    prev_s = rt.set_decode_split(split)
    try:
        c = Case(rt, 0x1A6E, 3, 32, 8, 128, [700, 450, 3000], 1, theta=5e5, quant=quant,
                 kv_dtype="bf16", permute_pages=True, k_transform=jump,
                 v_transform=lambda rng, v: v * np.float32(vscale))
        q = c.query("bf16")
        got = c.step_fused(q, "bf16")
        c.check_codes(seqs=[1])
        ref = c.oracle_attend(q)
        assert np.isfinite(got).all()
        wabs, rep = decode_weight_bounds(c, q)
        r = assert_close_decode_bound(got, ref, wabs, rep, "decode, large V")
        log(f"  worst err / bound {r:.4f}")
    finally:
        rt.set_decode_split(prev_s)


def test_decode_first_token_equals_v(rt):
    """One visible key: the output is that key's dequantised V (cf. the
    reference's test_gpu_gqa_first_token_no_history)."""
    log("decode first token")
    c = Case(rt, 51, 2, 8, 2, 128, [0, 0], 1)
    c.step_kv()
    q = c.query()
    got = c.gpu_decode(q)
    _, vd = c.ocache.dequant()
    for b in range(2):
        for hq in range(8):
            np.testing.assert_allclose(got[b, 0, hq * 128:(hq + 1) * 128], vd[b, hq // 4, 0],
                                       atol=1e-5, rtol=1e-5)


def test_decode_options(rt):
    log("decode: no rotary / interleaved / explicit scale")
    for rot, inter, scale in [(False, False, None), (True, True, None), (True, False, 0.05)]:
        c = Case(rt, 61, 2, 16, 4, 64, [200, 90], 1, do_rotary=rot, interleaved=inter)
        c.step_kv()
        q = c.query()
        assert_close(c.gpu_decode(q, scale=scale), c.oracle_attend(q, scale), f"{rot} {inter} {scale}")


def test_decode_ragged_paged_batch(rt):
    """64 sequences, seeded uniform lengths, 16-token pages, permuted page table."""
    log("decode ragged: 64 seqs, lengths U[16,1500], permuted pages")
    rng = np.random.default_rng(0x5A1A0003)
    lens = rng.integers(16, 1500, size=64).astype(np.int32)
    c = Case(rt, 71, 64, 32, 8, 128, lens, 1, theta=5e5, permute_pages=True)
    c.step_kv()
    q = c.query()
    assert_close(c.gpu_decode(q), c.oracle_attend(q), "ragged decode")


@pytest.mark.parametrize("merge", [0, 1])
@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
def test_decode_ragged_balanced_splits(rt, quant, merge):
    """Ragged batches deal each sequence's tiles evenly to its splits and hand
    the work items to the sequences with the longest splits first (batches of
    up to 256 sequences; the order rides in the kernel arguments). 300
    sequences (past the ordered limit: scan order) and 40 (ordered), lengths
    from 1 to 1200 tokens, split 256 (1 to 5 splits each, lengths like 257 and
    513 that would leave a one-token remainder), merged by the combine kernel
    (0) and in-kernel (1)."""
    log(f"decode ragged balanced splits quant={quant} merge={merge}")
    prev_s = rt.set_decode_split(256)
    prev_m = rt.set_decode_merge(merge)
    try:
        for n, seed in ((300, 0xBA1A), (40, 0xBA1B)):
            lens = np.random.default_rng(seed).integers(1, 1200, size=n).astype(np.int32)
            lens[:4] = [256, 512, 257, 1]
            c = Case(rt, seed, n, 8, 2, 64 if quant == S.KV_INT8 else 128, lens - 1, 1,
                     theta=1e4, quant=quant, permute_pages=True)
            q = c.query("bf16")
            got = c.step_fused(q, "bf16")
            assert_close(got, c.oracle_attend(q), f"ragged {n} sequences")
    finally:
        rt.set_decode_split(prev_s)
        rt.set_decode_merge(prev_m)


def test_decode_llama_layer_full_size(rt):
    """Full Llama-3-8B decode layer: B=16, 8k context, bf16 Q, int8 KV."""
    log("decode full size: B=16 ctx 8192 32Q/8KV D=128")
    c = Case(rt, 0x5A1A0001, 16, 32, 8, 128, [8191] * 16, 1, theta=5e5)
    c.step_kv()
    q = c.query("bf16")
    got = c.gpu_decode(q, "bf16")
    ref = c.oracle_attend(q)
    err = assert_close(got, ref, "c2 decode")
    log(f"  max abs err {err:.2e}, worst err/tol {err_tol_ratio(got, ref):.4f}")
    c.check_codes(seqs=[0, 15])


@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
def test_decode_bf16_output(rt, quant):
    """Attention output in bf16 (the reference's GPU GQA returns Q's dtype,
    attention.rs:835 and :877-901): the Llama-3-8B layer shape with 8k
    contexts (4 sequences), the fused step and the no-alloc step with bf16
    Q and bf16 output, against the f32 oracle within the tolerance widened
    by bf16 rounding; the decoded step's codes stay bit-exact. Split merges
    in-kernel (uniform) and through the combine kernel (ragged)."""
    log(f"decode bf16 output: quant {quant}")
    from _gpu_util import bf16_tol_close
    c = Case(rt, 0x5A1A0B16, 4, 32, 8, 128, [8191] * 4, 1, theta=5e5, quant=quant,
             kv_dtype="bf16", extra_tokens=3)
    q = c.query("bf16")
    got = c.step_fused(q, "bf16", out_dtype="bf16")
    ref = c.oracle_attend(q)
    r = bf16_tol_close(got, ref, "bf16 fused step")
    log(f"  uniform 8k: worst err/tol {r:.4f}")
    c.check_codes(seqs=[2])
    c.cache.advance()
    # ragged lengths: the combine kernel's store
    c.cache.set_seq_lens(np.array([8192, 3000, 777, 5000], np.int32))
    c.ocache.seq_len = np.array([8192, 3000, 777, 5000], np.int32)
    q = c.query("bf16")
    got = c.step_fused(q, "bf16", out_dtype="bf16")
    r = bf16_tol_close(got, c.oracle_attend(q), "bf16 fused step, ragged")
    log(f"  ragged: worst err/tol {r:.4f}")


def test_prefill_bf16_output(rt):
    """The prefill chunk at its workload's per-sequence shape (32Q/8KV, 2048
    new tokens over 6144 cached, bf16 Q/K/V), one sequence, with bf16 output:
    bit for bit the f32 output rounded to nearest even (prefill is
    deterministic), and within the bf16-widened tolerance of the oracle on
    sampled rows."""
    import copy
    from _gpu_util import bf16_tol_close, to_bf16_f32
    log("prefill bf16 output: B=1 past 6144 new 2048")
    c = Case(rt, 0x5A1A0B17, 1, 32, 8, 128, [6144], 2048, theta=5e5, kv_dtype="bf16")
    c.step_kv()
    q = c.query("bf16")
    got32 = c.gpu_prefill(q, "bf16")
    got16 = c.gpu_prefill(q, "bf16", out_dtype="bf16")
    np.testing.assert_array_equal(got16.view(np.uint32), to_bf16_f32(got32).view(np.uint32))
    deq = c.ocache.dequant()
    for i in [0, 1000, 2047]:
        oc = copy.copy(c.ocache)
        oc.seq_len = np.array([6144 + i + 1], dtype=np.int32)
        ref = oc.attend(q[:, i:i + 1], 32, c.cos, c.sin, deq=deq)
        bf16_tol_close(got16[:, i:i + 1], ref, f"bf16 prefill row {i}")


def test_output_dtype_errors(rt):
    """An output dtype other than f32/bf16 is UNSUPPORTED at every attention
    entry point."""
    import torch
    c = Case(rt, 0x0D7E, 1, 8, 2, 64, [40], 1)
    c.step_kv()
    q = dev(c.query())
    for bad in (torch.float16,):
        out = torch.zeros((1, 1, 8 * 64), dtype=bad, device="cuda")
        with pytest.raises(S.SaiError) as e:
            c.cache.decode(0, q, out, 1, 8, c.cos_d, c.sin_d, c.cos.shape[0])
        assert e.value.status == -3 and "output dtype" in str(e.value)
        with pytest.raises(S.SaiError) as e:
            c.cache.prefill(0, q, out, 1, 1, 8, c.cos_d, c.sin_d, c.cos.shape[0])
        assert e.value.status == -3


# ------------------------------------------------------------ int4 decode ---
@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (16, 2)])
def test_decode_int4_groups(rt, hq, hkv):
    log(f"decode int4 group {hq // hkv}: hq={hq} hkv={hkv}, outlier K, permuted pages")
    c = Case(rt, 0x1400 + hq, 3, hq, hkv, 128, [300, 129, 17], 1, theta=5e5, quant=S.KV_INT4,
             k_transform=outlier_student_t, permute_pages=True)
    c.step_kv()
    q = c.query()
    assert_close(c.gpu_decode(q), c.oracle_attend(q), f"int4 group {hq // hkv}")


def test_decode_int4_options(rt):
    log("decode int4: no rotary / interleaved / explicit scale / bf16")
    for rot, inter, scale, dt in [(False, False, None, "f32"), (True, True, None, "bf16"),
                                  (True, False, 0.05, "f32")]:
        c = Case(rt, 0x1410, 2, 16, 4, 128, [200, 90], 1, quant=S.KV_INT4, do_rotary=rot,
                 interleaved=inter, kv_dtype=dt)
        c.step_kv()
        q = c.query(dt)
        assert_close(c.gpu_decode(q, dt, scale=scale), c.oracle_attend(q, scale),
                     f"int4 {rot} {inter} {scale} {dt}")


def test_decode_int4_first_token_equals_v(rt):
    log("decode int4 first token")
    c = Case(rt, 0x1420, 2, 8, 2, 128, [0, 0], 1, quant=S.KV_INT4)
    c.step_kv()
    q = c.query()
    got = c.gpu_decode(q)
    _, vd = c.ocache.dequant()
    for b in range(2):
        for hq in range(8):
            np.testing.assert_allclose(got[b, 0, hq * 128:(hq + 1) * 128], vd[b, hq // 4, 0],
                                       atol=2e-3, rtol=1e-3)


@pytest.mark.parametrize("split", [64, 1024])
def test_decode_int4_split_merge(rt, split):
    log(f"decode int4 split merge split={split}")
    c = Case(rt, 0x1430, 3, 32, 8, 128, [3000, 1, 640], 1, quant=S.KV_INT4,
             k_transform=outlier_student_t, permute_pages=True)
    prev = rt.set_decode_split(split)
    try:
        c.step_kv()
        q = c.query()
        ref = c.oracle_attend(q)
        for _ in range(2):
            assert_close(c.gpu_decode(q), ref, f"int4 split {split}")
    finally:
        rt.set_decode_split(prev)


@pytest.mark.parametrize("split", [64, 4096])
def test_decode_int4_fused_step(rt, split):
    """Fused int4 step: the decode kernel appends the token (V nibble shared
    with the neighbouring slot) and attends; codes bit-exact with the oracle."""
    log(f"fused int4 decode step split={split}")
    prev_s = rt.set_decode_split(split)
    try:
        c = Case(rt, 0x1440, 3, 32, 8, 128, [700, 4, 4100], 1, theta=5e5, kv_dtype="bf16",
                 quant=S.KV_INT4, k_transform=outlier_student_t, permute_pages=True,
                 extra_tokens=2)
        for step in range(3):
            q = c.query("bf16")
            got = c.step_fused(q, "bf16")
            assert_close(got, c.oracle_attend(q), f"fused int4 step {step}")
            c.check_codes(seqs=[1])
            c.cache.advance()
    finally:
        rt.set_decode_split(prev_s)


def test_decode_int4_long_context_full_size(rt):
    """Long-context int4 decode at full size: B=4, 32k context, 32Q/8KV, K
    Student-t with x20 outlier channels."""
    log("decode int4 full size: B=4 ctx 32768 32Q/8KV D=128")
    c = Case(rt, 0x5A1A0002, 4, 32, 8, 128, [32767] * 4, 1, theta=5e5, quant=S.KV_INT4,
             k_transform=outlier_student_t)
    c.step_kv()
    q = c.query("bf16")
    got = c.gpu_decode(q, "bf16")
    ref = c.oracle_attend(q)
    err = assert_close(got, ref, "c3 decode")
    log(f"  max abs err {err:.2e}")
    c.check_codes(seqs=[3])


# ---------------------------------------------------------------- prefill ---
@pytest.mark.parametrize("hq,hkv,d,past,new,qd", [
    (8, 2, 64, [100, 37], 70, "f32"),
    (32, 8, 128, [300, 0], 200, "bf16"),
    (8, 8, 128, [64, 17], 130, "f32"),
    (16, 2, 128, [5, 250], 33, "f32"),
])
def test_prefill_small(rt, hq, hkv, d, past, new, qd):
    log(f"prefill hq={hq} hkv={hkv} d={d} past={past} new={new} {qd}")
    c = Case(rt, 81 + new, len(past), hq, hkv, d, past, new, theta=5e5, permute_pages=True,
             kv_dtype=qd)
    c.step_kv()
    c.check_codes()
    q = c.query(qd)
    got = c.gpu_prefill(q, qd)
    ref = c.oracle_attend(q)
    assert_close(got, ref, "prefill")


def test_prefill_chunk_full_size_sampled(rt):
    """B=2, 2048 new tokens over 6144 cached, 32Q/8KV: append + prefill at full
    size; outputs checked on sampled query rows (oracle per row)."""
    import copy

    log("prefill full size: B=2 past 6144 new 2048")
    c = Case(rt, 0x5A1A0004, 2, 32, 8, 128, [6144, 6144], 2048, theta=5e5, kv_dtype="bf16")
    c.step_kv()
    q = c.query("bf16")
    got = c.gpu_prefill(q, "bf16")
    c.check_codes(seqs=[1])
    deq = c.ocache.dequant()
    for i in [0, 1, 63, 64, 777, 1500, 2046, 2047]:
        oc = copy.copy(c.ocache)
        oc.seq_len = np.array([6144 + i + 1] * 2, dtype=np.int32)
        ref = oc.attend(q[:, i:i + 1], 32, c.cos, c.sin, deq=deq)
        assert_close(got[:, i:i + 1], ref, f"prefill row {i}")


@pytest.mark.parametrize("quant,hq,hkv,d,past,new,qd", [
    (S.KV_INT4, 16, 4, 128, [300, 0], 150, "bf16"),
    (S.KV_INT4, 8, 2, 64, [100, 37], 70, "f32"),
    (S.KV_INT4, 32, 8, 128, [64, 640], 33, "f32"),
    (S.KV_INT8, 16, 4, 128, [300, 0], 150, "bf16"),
    (S.KV_INT8, 8, 2, 64, [100, 37], 70, "f32"),
])
def test_prefill_outlier_keys(rt, quant, hq, hkv, d, past, new, qd):
    """Prefill with K carrying x20 outlier channels (Student-t elsewhere), whose
    largest score terms are in the hundreds: the split (hi + lo) query and, for
    int4, the split dequantised K keep the outputs within tolerance. int4 codes
    and group parameters bit-exact; ragged past lengths."""
    log(f"prefill outlier K quant={quant} hq={hq} hkv={hkv} d={d} past={past} new={new} {qd}")

    def outliers(rng, k):
        b, n, hd = k.shape
        t = rng.standard_t(3, size=k.shape).astype(np.float32).reshape(b, n, hd // d, d)
        t[..., [5, 17, d - 3]] *= 20.0
        return t.reshape(b, n, hd)

    c = Case(rt, 131 + new, len(past), hq, hkv, d, past, new, theta=5e5, quant=quant,
             permute_pages=True, kv_dtype=qd, k_transform=outliers)
    c.step_kv()
    c.check_codes()
    q = c.query(qd)
    got = c.gpu_prefill(q, qd)
    ref = c.oracle_attend(q)
    log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
    err = assert_close(got, ref, "outlier-K prefill")
    log(f"  max abs err {err:.2e}")


@pytest.mark.parametrize("quant,vscale", [
    (S.KV_INT8, 1.0), (S.KV_INT8, 1.0e5), (S.KV_INT8, 1.0e7), (S.KV_INT4, 1.0e4),
])
def test_prefill_reference_moves(rt, quant, vscale):
    """Prefill whose weights leave the fast path's bounds mid-sequence: keys
    at past positions 300-339 are scaled x6, so their scores rise tens of log2
    units above the reference point the first tiles set. With vscale 1e5 and
    1e7 the V rows reach |v| ~ 4e5 and 4e7 (int4: 1e4, as its binary16 zero
    point allows): int8 tiles with V scales above
    the large-V threshold go to the precise pass (binary16 hi + lo weights
    normalised by a power of two, so nothing overflows binary16; 1e7 put
    p * s_v past 65504 before), int4 V is staged scaled by 2^-5. Codes
    bit-exact. The outputs cancel to ~1e3 against |v| ~ 4e5, where the
    oracle's own expf_approx (3.5e-5 relative) already moves them by more than
    2e-3, so large V is checked against the weighted bound
    2e-3 + 1e-2|ref| + kappa sum p|v| / sum p: kappa 2^-12 for the precise
    int8 pass, 2^-9 for int4 (binary16 weights and V values)."""
    log(f"prefill reference moves: quant {quant}, keys x6 at 300-339, V x{vscale:g}")

    def jump(rng, k):
        if k.shape[1] >= 340:
            k[:, 300:340] *= 6.0
        return k

    c = Case(rt, 0x5E77, 2, 16, 4, 128, [700, 450], 130, theta=5e5, quant=quant,
             permute_pages=True, k_transform=jump,
             v_transform=lambda rng, v: v * np.float32(vscale))
    c.step_kv()
    c.check_codes()
    q = c.query("f32")
    got = c.gpu_prefill(q, "f32")
    ref = c.oracle_attend(q)
    assert np.isfinite(got).all()
    if vscale == 1.0:
        log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
        assert_close(got, ref, "prefill, reference moves")
        return
    kappa = 2.0 ** -12 if quant == S.KV_INT8 else 2.0 ** -9
    r = assert_close_weighted(got, ref, weighted_abs_v(c, q), kappa, "prefill, large V")
    log(f"  worst err / weighted bound {r:.4f}")


@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
def test_prefill_first_key_far_below(rt, quant):
    """Row 0 of a fresh prompt sees one key; its query is -20 x that key, so
    its only score is ~ -330 (log2 units). The reference point then moves
    down by 330 on the row's first keys, where exp2(330) is inf: the row must
    still come out as v0 (it came out NaN when the rescale of the empty
    accumulator was exp2(-lead)). Also rows at a window edge that see only
    that key."""
    log(f"prefill first key far below: quant {quant}")
    c = Case(rt, 0xF1F0, 2, 8, 2, 128, [0, 0], 64, theta=1e4, quant=quant)
    c.step_kv()
    c.check_codes()
    q = c.query("f32")
    k0 = c.ocache.dequant()[0][:, :, 0, :]  # [B, Hkv, D] (position 0: RoPE is the identity)
    for b in range(2):
        for h in range(8):
            q[b, 0, h * 128:(h + 1) * 128] = -20.0 * k0[b, h // 4]
    got = c.gpu_prefill(q, "f32")
    ref = c.oracle_attend(q)
    assert np.isfinite(got).all(), "NaN/inf in the prefill output"
    assert_close(got, ref, "prefill, first key far below")
    got_w = c.gpu_prefill(q, "f32", window=1)
    ref_w = c.oracle_attend(q, mask_window=1)
    assert np.isfinite(got_w).all()
    assert_close(got_w, ref_w, "prefill, window 1")


# ------------------------------------------------------------- introspection ---
def test_decode_kernel_timing_ring(rt):
    """sai_set_decode_timing / sai_decode_kernel_times: events around the decode
    kernel of back-to-back calls, oldest first, at most the slot count."""
    log("decode kernel timing ring")
    c = Case(rt, 0x7100, 2, 8, 2, 128, [700, 300], 1)
    c.step_kv()
    q = c.query()
    prev = rt.set_decode_timing(3)
    try:
        assert rt.decode_kernel_times(8) == []
        for _ in range(5):
            c.gpu_decode(q)
        t = rt.decode_kernel_times(8)
        assert len(t) == 3 and all(0.0 < x < 1e5 for x in t), t
    finally:
        rt.set_decode_timing(prev)
    assert rt.decode_kernel_times(8) == []


@pytest.mark.parametrize("quant", [S.KV_INT8, S.KV_INT4])
def test_split_merge_handoff_repeated(rt, quant):
    """The in-kernel split merge hands partials between workgroups on different XCDs
    (agent-scope stores, a wait for their completion, then the ticket; the last
    ticket's holder loads them). With 64-token splits this 4 x 8k batch makes up to 128
    splits per (sequence, kv head), 3824 workgroups: 30 launches with the fixed tile order must
    give the same bits every time (a partial read before its store landed would change
    an output), and agree with the combine kernel's merge and the oracle within
    tolerance."""
    log(f"split merge handoff, 30 launches, split 64, quant {quant}")
    c = Case(rt, 0x4A4D0FF + quant, 4, 32, 8, 128, [8191, 8191, 6000, 8191], 1, theta=5e5,
             kv_dtype="bf16", quant=quant)
    c.step_kv()
    q = c.query("bf16")
    prev_r = rt.set_decode_reproducible(1)
    prev_s, prev_m = rt.set_decode_split(64), rt.set_decode_merge(1)
    try:
        outs = [c.gpu_decode(q, "bf16") for _ in range(30)]
        rt.set_decode_merge(0)
        comb = c.gpu_decode(q, "bf16")
    finally:
        rt.set_decode_reproducible(prev_r)
        rt.set_decode_split(prev_s)
        rt.set_decode_merge(prev_m)
    wg, split = rt.last_decode_shape()
    assert split == 64 and wg == sum((n + 1 + 63) // 64 for n in c.past_lens) * 8
    for i, o in enumerate(outs[1:], 1):
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), f"launch {i} differs"
    assert np.abs(outs[0] - comb).max() <= 1e-4
    assert_close(outs[0], c.oracle_attend(q), "in-kernel merge of 128 splits")


@pytest.mark.parametrize("merge", [1, 0])
def test_decode_reproducible_tile_order(rt, merge):
    """With the fixed tile order (sai_set_decode_reproducible) repeated decode
    calls over the same cache give bit-identical outputs (the Llama-3-8B layer
    shape, 4 x 8k, many splits merged in-kernel and by the combine kernel),
    within tolerance of the oracle; the run-time order stays within tolerance
    too."""
    log(f"decode reproducible tile order, merge {merge}")
    c = Case(rt, 0x5A1A0F1E, 4, 32, 8, 128, [8191, 8191, 5000, 8191], 1, theta=5e5,
             kv_dtype="bf16")
    c.step_kv()
    q = c.query("bf16")
    ref = c.oracle_attend(q)
    prev_r = rt.set_decode_reproducible(1)
    prev_s, prev_m = rt.set_decode_split(512), rt.set_decode_merge(merge)
    try:
        outs = [c.gpu_decode(q, "bf16") for _ in range(4)]
        rt.set_decode_reproducible(0)
        dyn = c.gpu_decode(q, "bf16")
    finally:
        rt.set_decode_reproducible(prev_r)
        rt.set_decode_split(prev_s)
        rt.set_decode_merge(prev_m)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), "fixed order differs"
    assert_close(outs[0], ref, "fixed tile order")
    assert_close(dyn, ref, "run-time tile order")
    log(f"  fixed vs run-time: max |diff| {np.abs(outs[0] - dyn).max():.3e}")
