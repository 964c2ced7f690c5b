"""Fidelity of the GPU TurboQuant attention against uncompressed attention.

1. The reference's integration_synthetic_gqa_compressed_vs_uncompressed
   (onnx-rt/src/kv_compression.rs:1752-1829) through the GPU cache: the same
   32 xorshift64 rows of head_dim 64 at 4 bits + QJL, seed 42. read_k on the
   GPU equals the oracle's decode bit for bit, so the reference's logits
   q . read_k pass its bar (max error / mean |logit| < 1.0) exactly as on the
   CPU; the GPU's attention_logits (the decode path's estimator: the query
   encoded by the same quantiser, plus the QJL correction) must pass the same
   bar against the uncompressed logits.
2. At the tq4 workload's shape (16 sequences x 8192 positions, 32 query / 8
   kv heads, head_dim 128, 4 bits + QJL, bf16 queries), sampled (sequence,
   kv head) pairs: the distance of sai_tqcache_attend's output from
   softmax(scale q . read_k) read_v (raw query over the decoded cache) and
   from softmax(scale q . k) v (no compression), logged. The estimator
   quantises the query as well, so it may not be further from the
   uncompressed output than a fixed fraction of the output's own size.
"""
import numpy as np
import pytest

import oracle as O
import smallaios_amd as S
from _gpu_util import log
from test_oracle_tq_fidelity import BITS, DIM, SEED, SEQ, reference_rows

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    r = S.Runtime(0)
    yield r
    r.close()


def test_reference_integration_on_gpu(rt):
    import torch
    log("tq fidelity: the reference's compressed-vs-uncompressed logits, 32 x 64, 4 bit + QJL")
    k, v, q = reference_rows()
    c = S.TqCache(rt, 1, 1, DIM, BITS, True, 1, SEQ, seed=SEED)
    try:
        c.write(0, torch.from_numpy(k[None]).cuda(), torch.from_numpy(v[None]).cuda(), 1, SEQ)
        c.advance()
        k_read, _ = c.read(0, 0, 0, 0, SEQ)
        sg = O.tq_signs(O.tq_head_seed(SEED, 0, 1, 0), DIM)
        enc = O.tq_write_rows(k, BITS, sg, True)
        want = np.stack([O.tq_decode(enc[0][t], DIM, BITS, enc[1][t], enc[2][t], sg)
                         for t in range(SEQ)])
        assert np.array_equal(k_read.view(np.uint32), want.view(np.uint32))
        true = k.astype(np.float64) @ q.astype(np.float64)
        mean = np.abs(true).mean() + 1e-6
        rel_read = np.abs(true - k_read.astype(np.float64) @ q).max() / mean
        logits = torch.zeros((1, SEQ), device="cuda")
        c.attention_logits(0, torch.from_numpy(q[None, None]).cuda(), logits, SEQ, 1, 1)
        torch.cuda.synchronize()
        est = logits.cpu().numpy()[0].astype(np.float64)
        rel_est = np.abs(true - est).max() / mean
        log(f"  relative logit error: raw q . read_k {rel_read:.4f}, GPU estimator {rel_est:.4f}")
        assert rel_read < 1.0 and rel_est < 1.0
        ref_est = O.tq_attention_logits(q[None, :], BITS, True, sg, enc)[0]
        np.testing.assert_allclose(est, ref_est, rtol=1e-4, atol=1e-4)
    finally:
        c.close()


def softmax_attend(q, k, v, scale):
    """softmax(scale q k^T) v in f64; q [G, D], k/v [T, D]."""
    s = (q.astype(np.float64) @ k.astype(np.float64).T) * scale
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return p @ v.astype(np.float64)


def test_attend_vs_uncompressed_tq4_shape(rt):
    import torch
    log("tq fidelity at the tq4 shape: attend vs raw-query attention over read_k/read_v")
    batch, heads, group, d, bits, ctx = 16, 8, 4, 128, 4, 8192
    nh = heads * group
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x7A4F1D)
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
        q = torch.randn((batch, 1, nh * d), generator=gen, device="cuda").to(torch.bfloat16)
        out = torch.zeros((batch, 1, nh * d), device="cuda")
        c.attend(0, q, out, batch, nh)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(batch, nh, d).astype(np.float64)
        qq = q.float().cpu().numpy().reshape(batch, nh, d)
        k_all = torch.cat(ks, dim=1)
        v_all = torch.cat(vs, dim=1)
        scale = S.default_scale(d)
        worst_read, worst_true, worst_read_vs_true = 0.0, 0.0, 0.0
        for b, h in [(0, 0), (3, 2), (7, 5), (12, 1), (15, 7)]:
            kr, vr = c.read(0, b, h, 0, ctx)
            kt = k_all[b, :, h * d:(h + 1) * d].cpu().numpy()
            vt = v_all[b, :, h * d:(h + 1) * d].cpu().numpy()
            qg = qq[b, h * group:(h + 1) * group]
            over_read = softmax_attend(qg, kr, vr, scale)
            exact = softmax_attend(qg, kt, vt, scale)
            g = got[b, h * group:(h + 1) * group]
            size = np.abs(exact).max()
            e_read = np.abs(g - over_read).max() / size
            e_true = np.abs(g - exact).max() / size
            e_rt = np.abs(over_read - exact).max() / size
            log(f"  b={b} h={h}: max|out - attn(read_k, read_v)| / max|exact| {e_read:.4f}; "
                f"vs uncompressed {e_true:.4f}; raw-query attn over read_k/read_v vs "
                f"uncompressed {e_rt:.4f}")
            worst_read = max(worst_read, e_read)
            worst_true = max(worst_true, e_true)
            worst_read_vs_true = max(worst_read_vs_true, e_rt)
        log(f"  worst: vs read_k/read_v {worst_read:.4f}, vs uncompressed {worst_true:.4f} "
            f"(raw query over read_k/read_v: {worst_read_vs_true:.4f})")
        assert worst_true < 0.5 and worst_read < 0.5
    finally:
        c.close()
