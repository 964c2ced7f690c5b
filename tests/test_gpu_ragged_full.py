"""The ragged continuous-batch decode at its configured lengths.

64 sequences with lengths U[128, 16384] (seed 0x5A1A0003, the bench's own
draw: numpy default_rng(seed).integers(128, 16385, 64)), 32 query / 8 kv heads,
head_dim 128, int8 KV in 16-token pages behind a randomly permuted page table,
one fused decode step (sai_gqa_with_cache) at the automatic split, which cuts
the longest sequences into up to 6 pieces of 3072 tokens merged by the
8-wide combine. The whole batch runs on the GPU; the shortest, the longest and
six more sampled sequences are checked against the oracle (a cache holding
only those sequences, built from the same K/V values), and the shortest and
longest sequences' codes bit for bit.

Reference semantics: scaled_dot_product_attention
(onnx-rt/src/ops/microsoft.rs:380-438) over the dequantised cache.
"""
import numpy as np
import pytest

import oracle as O
import smallaios_amd as S
from _gpu_util import assert_close, err_tol_ratio, log

pytestmark = pytest.mark.gpu

SEED = 0x5A1A0003
B, HQ, HKV, D, THETA = 64, 32, 8, 128, 5e5


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    r = S.Runtime(0)
    yield r
    r.close()


def test_decode_ragged_full_lengths(rt):
    import torch

    lens = np.random.default_rng(SEED).integers(128, 16384 + 1, size=B).astype(np.int64)
    past = (lens - 1).astype(np.int32)
    rng = np.random.default_rng(SEED + 1)
    order = np.argsort(lens)
    others = rng.choice(order[1:-1], size=6, replace=False)
    sampled = np.array([order[0], order[-1], *others], dtype=np.int64)
    log(f"ragged full lengths: 64 seqs, sum {int(lens.sum())}, min {lens.min()}, "
        f"max {lens.max()}; sampled {sampled.tolist()} lens {lens[sampled].tolist()}")

    pages = (int(lens.max()) + S.PAGE_TOKENS - 1) // S.PAGE_TOKENS
    cos, sin = S.rope_tables(int(lens.max()) + 1, D, THETA)
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    cache = S.KvCache(rt, 1, HKV, D, B * pages, B, pages, S.KV_INT8)
    ids = np.random.default_rng(SEED + 2).permutation(B * pages).astype(np.int32)
    cache.set_page_table(ids.reshape(B, pages))

    # every sequence gets max(past) tokens (generated on the device), then the
    # lengths are cut to past[b]; the sampled sequences' rows are kept on the
    # host for the oracle
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    pmax = int(past.max())
    ns = len(sampled)
    hk = np.zeros((ns, pmax, HKV * D), np.float32)
    hv = np.zeros_like(hk)
    sel = torch.from_numpy(sampled).cuda()
    done = 0
    while done < pmax:
        n = min(2048, pmax - done)
        k = torch.randn((B, n, HKV * D), generator=gen, device="cuda").to(torch.bfloat16)
        v = torch.randn((B, n, HKV * D), generator=gen, device="cuda").to(torch.bfloat16)
        cache.append(0, k, v, B, n, cos_d, sin_d, cos.shape[0])
        cache.advance()
        hk[:, done:done + n] = k.index_select(0, sel).float().cpu().numpy()
        hv[:, done:done + n] = v.index_select(0, sel).float().cpu().numpy()
        done += n
    cache.set_seq_lens(past)

    oc = O.LogicalCache(ns, HKV, D, int(lens[sampled].max()), O.INT8)
    oc.append(hk[:, :int(past[sampled].max())], hv[:, :int(past[sampled].max())], cos, sin)
    oc.seq_len = past[sampled].astype(np.int32)
    del hk, hv

    # the step: new K/V and Q for every sequence, fused append + decode
    kn = torch.randn((B, 1, HKV * D), generator=gen, device="cuda").to(torch.bfloat16)
    vn = torch.randn((B, 1, HKV * D), generator=gen, device="cuda").to(torch.bfloat16)
    q = torch.randn((B, 1, HQ * D), generator=gen, device="cuda").to(torch.bfloat16)
    out = torch.zeros((B, 1, HQ * D), dtype=torch.float32, device="cuda")
    cache.decode_with_cache(0, q, kn, vn, out, B, HQ, cos_d, sin_d, cos.shape[0])
    torch.cuda.synchronize()
    wg, split = rt.last_decode_shape()
    n_splits = (lens + split - 1) // split
    log(f"  automatic split {split} tokens, {wg} workgroups, "
        f"up to {int(n_splits.max())} splits per sequence")
    assert split == 3072 and int(n_splits.max()) == 6 and wg == int(n_splits.sum()) * HKV

    oc.append(kn.index_select(0, sel).float().cpu().numpy(),
              vn.index_select(0, sel).float().cpu().numpy(), cos, sin)
    qs = q.index_select(0, sel).float().cpu().numpy()
    ref = oc.attend(qs, HQ, cos, sin)
    got = out.index_select(0, sel).cpu().numpy()
    log(f"  worst err/tol {err_tol_ratio(got, ref):.4f}")
    assert_close(got, ref, "ragged full lengths")

    # codes of the shortest sequence, and the last 64 tokens of the longest
    for i, t0 in ((0, 0), (1, int(lens[sampled[1]]) - 64)):
        bsel = int(sampled[i])
        n = int(lens[bsel]) - t0
        for h in range(HKV):
            kc, vc, ks, vs = cache.read(0, bsel, h, t0, n)
            np.testing.assert_array_equal(kc, oc.k_codes[i, h, t0:t0 + n])
            np.testing.assert_array_equal(vc, oc.v_codes[i, h, t0:t0 + n])
            np.testing.assert_array_equal(ks.view(np.uint32),
                                          oc.k_scale[i, h, t0:t0 + n].view(np.uint32))
            np.testing.assert_array_equal(vs.view(np.uint32),
                                          oc.v_scale[i, h, t0:t0 + n].view(np.uint32))
    cache.close()
