"""Shared helpers of the GPU parity tests: build the same quantised cache on
the GPU (through the C ABI) and in the oracle, then compare."""
from __future__ import annotations

import sys

import numpy as np

import oracle as O
import smallaios_amd as S

ATOL = 2e-3  # attention outputs: |gpu - ref| <= ATOL + RTOL * |ref|
RTOL = 1e-2


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def to_bf16_f32(x: np.ndarray) -> np.ndarray:
    """Round f32 -> bf16 (RNE, as the reference's f32_to_bf16) and back to f32."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def _torch_dtype(name):
    import torch
    return {"f32": torch.float32, "bf16": torch.bfloat16}[name]


def bf16_tol_close(got, ref, what=""):
    """A bf16 attention output against the f32 oracle: the 2e-3 abs + 1e-2
    rel tolerance widened by bf16's round-to-nearest (2^-9 of the value, on
    both sides)."""
    err = np.abs(got - ref)
    tol = ATOL + (RTOL + 2.0 ** -8) * np.abs(ref)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside the bf16 "
                             f"tolerance; worst at {i}: got {got[i]}, ref {ref[i]}")
    return float((err / tol).max())


def dev(x: np.ndarray, dtype="f32"):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    if dtype == "bf16":
        t = t.to(torch.bfloat16)
    return t.contiguous()


def outlier_student_t(rng, k):
    """K of the long-context int4 workload: Student-t (df 3) with four fixed
    outlier channels per head scaled x20."""
    b, n, hd = k.shape
    t = rng.standard_normal(k.shape).astype(np.float32) / np.sqrt(
        rng.chisquare(3, size=k.shape) / 3).astype(np.float32)
    t = t.reshape(b, n, hd // 128, 128)
    t[..., [7, 31, 64, 100]] *= 20.0
    return t.reshape(b, n, hd).astype(np.float32)


class Case:
    """One cache (GPU + oracle) with `batch` sequences.

    past_lens: committed lengths before the step under test; the past K/V is
    appended by the HIP append kernel in one prefill-style call (max(past)
    tokens per sequence) and then truncated per sequence with set_seq_lens.
    """

    def __init__(self, rt, seed, batch, hq, hkv, d, past_lens, new_tokens, theta=10000.0,
                 quant=S.KV_INT8, kv_dtype="f32", permute_pages=False, do_rotary=True,
                 interleaved=False, k_transform=None, extra_pages=3, max_pages_per_seq=None,
                 extra_tokens=0, v_transform=None):
        self.rng = np.random.default_rng(seed)
        self.rt = rt
        self.batch, self.hq, self.hkv, self.d = batch, hq, hkv, d
        self.past_lens = np.asarray(past_lens, dtype=np.int32)
        self.new_tokens = new_tokens
        self.quant = quant
        self.kv_dtype = kv_dtype
        self.do_rotary, self.interleaved = do_rotary, interleaved
        self.k_transform = k_transform
        self.v_transform = v_transform
        total = int(self.past_lens.max()) + new_tokens + extra_tokens
        self.t_cap = total
        self.max_pages = max_pages_per_seq or (total + S.PAGE_TOKENS - 1) // S.PAGE_TOKENS
        num_pages = batch * self.max_pages + extra_pages
        self.cos, self.sin = S.rope_tables(total + 8, d, theta)
        self.cos_d, self.sin_d = dev(self.cos), dev(self.sin)
        self.cache = S.KvCache(rt, 1, hkv, d, num_pages, batch, self.max_pages, quant)
        if permute_pages:
            ids = self.rng.permutation(num_pages)[: batch * self.max_pages]
        else:
            ids = np.arange(batch * self.max_pages)
        self.page_table = ids.astype(np.int32).reshape(batch, self.max_pages)
        self.cache.set_page_table(self.page_table)
        self.ocache = O.LogicalCache(batch, hkv, d, self.t_cap, quant)
        pmax = int(self.past_lens.max())
        if pmax > 0:
            k, v = self.kv(pmax)
            self.append_both(k, v)
            self.cache.advance()
            self.cache.set_seq_lens(self.past_lens)
            self.ocache.seq_len = self.past_lens.copy()

    def kv(self, n):
        shape = (self.batch, n, self.hkv * self.d)
        k = self.rng.standard_normal(shape, dtype=np.float32)
        v = self.rng.standard_normal(shape, dtype=np.float32)
        if self.k_transform is not None:
            k = self.k_transform(self.rng, k)
        if self.v_transform is not None:
            v = self.v_transform(self.rng, v)
        if self.kv_dtype == "bf16":
            k, v = to_bf16_f32(k), to_bf16_f32(v)
        return k, v

    def append_both(self, k, v):
        n = k.shape[1]
        self.cache.append(0, dev(k, self.kv_dtype), dev(v, self.kv_dtype), self.batch, n,
                          self.cos_d, self.sin_d, self.cos.shape[0], self.do_rotary,
                          self.interleaved)
        self.ocache.append(k, v, self.cos, self.sin, self.do_rotary, self.interleaved)

    def step_kv(self):
        """Append the step's new tokens (pending on the GPU)."""
        k, v = self.kv(self.new_tokens)
        self.append_both(k, v)

    def query(self, q_dtype="f32"):
        q = self.rng.standard_normal((self.batch, self.new_tokens, self.hq * self.d),
                                     dtype=np.float32)
        if q_dtype == "bf16":
            q = to_bf16_f32(q)
        return q

    def check_codes(self, seqs=None):
        """Bit-exact comparison of every stored code and scale."""
        lens = self.ocache.seq_len
        for b in (range(self.batch) if seqs is None else seqs):
            n = int(lens[b])
            for h in range(self.hkv):
                kc, vc, kp, vp = self.cache.read(0, b, h, 0, n)
                oc = self.ocache
                np.testing.assert_array_equal(kc, oc.k_codes[b, h, :n], err_msg=f"K codes b={b} h={h}")
                np.testing.assert_array_equal(vc, oc.v_codes[b, h, :n], err_msg=f"V codes b={b} h={h}")
                if self.quant == S.KV_INT8:
                    np.testing.assert_array_equal(kp.view(np.uint32), oc.k_scale[b, h, :n].view(np.uint32),
                                                  err_msg=f"K scales b={b} h={h}")
                    np.testing.assert_array_equal(vp.view(np.uint32), oc.v_scale[b, h, :n].view(np.uint32),
                                                  err_msg=f"V scales b={b} h={h}")
                else:
                    np.testing.assert_array_equal(kp, oc.k_sz[b, h, :n], err_msg=f"K params b={b} h={h}")
                    np.testing.assert_array_equal(vp, oc.v_sz[b, h, :n], err_msg=f"V params b={b} h={h}")

    def gpu_decode(self, q, q_dtype="f32", scale=None, window=0, out_dtype="f32"):
        import torch
        out = torch.zeros((self.batch, 1, self.hq * self.d), dtype=_torch_dtype(out_dtype),
                          device="cuda")
        self.cache.decode(0, dev(q, q_dtype), out, self.batch, self.hq, self.cos_d, self.sin_d,
                          self.cos.shape[0], self.do_rotary, self.interleaved, scale,
                          window=window)
        torch.cuda.synchronize()
        return out.float().cpu().numpy()

    def step_fused(self, q, q_dtype="f32", scale=None, window=0, out_dtype="f32"):
        """Append the step's token and attend in one launch (sai_gqa_with_cache)."""
        import torch
        k, v = self.kv(1)
        self.ocache.append(k, v, self.cos, self.sin, self.do_rotary, self.interleaved)
        out = torch.zeros((self.batch, 1, self.hq * self.d), dtype=_torch_dtype(out_dtype),
                          device="cuda")
        self.cache.decode_with_cache(0, dev(q, q_dtype), dev(k, self.kv_dtype),
                                     dev(v, self.kv_dtype), out, self.batch, self.hq, self.cos_d,
                                     self.sin_d, self.cos.shape[0], self.do_rotary,
                                     self.interleaved, scale, window=window)
        torch.cuda.synchronize()
        return out.float().cpu().numpy()

    def gpu_prefill(self, q, q_dtype="f32", scale=None, window=0, out_dtype="f32"):
        import torch
        out = torch.zeros((self.batch, self.new_tokens, self.hq * self.d),
                          dtype=_torch_dtype(out_dtype), device="cuda")
        self.cache.prefill(0, dev(q, q_dtype), out, self.batch, self.new_tokens, self.hq,
                           self.cos_d, self.sin_d, self.cos.shape[0], self.do_rotary,
                           self.interleaved, scale, window=window)
        torch.cuda.synchronize()
        return out.float().cpu().numpy()

    def oracle_attend(self, q, scale=None, layer_window=0, mask_window=0):
        return self.ocache.attend(q, self.hq, self.cos, self.sin, self.do_rotary,
                                  self.interleaved, scale, layer_window=layer_window,
                                  mask_window=mask_window)


def err_tol_ratio(got, ref):
    """max over elements of |got - ref| / (ATOL + RTOL |ref|): 1.0 is the edge
    of the tolerance."""
    return float((np.abs(got - ref) / (ATOL + RTOL * np.abs(ref))).max())


def outlier_keys(d, channels=(7, 31, 64, 100), factor=20.0):
    """k_transform: Student-t (df 3) keys with `channels` of every head of
    head_dim d scaled by `factor` (heavy tails plus the fixed outlier
    channels of real models' keys)."""

    def tf(rng, k):
        b, n, hd = k.shape
        t = rng.standard_t(3, size=k.shape).astype(np.float32).reshape(b, n, hd // d, d)
        t[..., list(channels)] *= np.float32(factor)
        return t.reshape(b, n, hd)

    return tf


def assert_close(got, ref, what=""):
    err = np.abs(got - ref)
    tol = ATOL + RTOL * np.abs(ref)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside {ATOL} abs / {RTOL} rel; "
            f"worst at {i}: got {got[i]}, ref {ref[i]}, max abs err {err.max():.3e}")
    return float(err.max())


def weighted_abs_v(case, q):
    """sum_t p_t |v_t| / sum_t p_t per output element: the oracle's attention
    with every dequantised V value replaced by its magnitude (the scale of
    the error that relative errors in the softmax weights can cause)."""
    kd, vd = case.ocache.dequant()
    return case.ocache.attend(q, case.hq, case.cos, case.sin, case.do_rotary, case.interleaved,
                              deq=(kd, np.abs(vd)))


def assert_close_weighted(got, ref, wabs, kappa, what=""):
    """|got - ref| <= ATOL + RTOL |ref| + kappa * sum p|v| / sum p.

    If the weights p_t of both results carry relative errors of at most e,
    their outputs sum p v / sum p differ by at most 2 e sum p|v| / sum p
    (first order), whatever V's magnitude; the fixed ATOL says nothing once
    |v| is large and the output cancels far below it. kappa = 2 e covers the
    oracle's degree-4 expf_approx (relative error below 3.5e-5) and the
    kernel's own weight rounding."""
    err = np.abs(got - ref)
    tol = ATOL + RTOL * np.abs(ref) + kappa * wabs
    ratio = float((err / tol).max())
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside the weighted bound (kappa "
            f"{kappa:.3g}); worst at {i}: got {got[i]}, ref {ref[i]}, sum p|v| {wabs[i]:.4g}")
    return ratio


def decode_weight_bounds(case, q):
    """Error scales of the decode kernels' softmax weights, per output element
    of a decode step (q [B, 1, Hq*D], pre-RoPE; the oracle cache already
    holds the step's token), from the oracle's codes with f64 weights:
      wabs = sum p|v| / sum p;
      rep  = what the kernel's weight representation can move the output by:
        int8: P' = p * s_v of each 64-token tile is held as hi + residual/254
              int8 terms against the tile's largest P', an error of at most
              max P' / 64516 per token, so
              rep = sum over tiles (max P' * sum_t |code_t|) / (64516 sum p);
        int4: P' = p * s_v(group) as binary16 (2^-11 relative) times the code:
              rep = 2^-11 sum p |v - z| / sum p."""
    B, Hq, D, Hkv = case.batch, case.hq, case.d, case.hkv
    G = Hq // Hkv
    oc = case.ocache
    L = oc.seq_len
    kd, vd = oc.dequant()
    scale = O.default_scale(D)
    qh = np.asarray(q, np.float32).reshape(B, 1, Hq, D).transpose(0, 2, 1, 3)
    wabs = np.zeros((B, Hq, D))
    rep = np.zeros((B, Hq, D))
    for b in range(B):
        n = int(L[b])
        qr = qh[b:b + 1]
        if case.do_rotary:
            qr = O.apply_rope(qr, case.cos, case.sin, [n - 1], case.interleaved)
        for h in range(Hq):
            kh = h // G
            s = kd[b, kh, :n].astype(np.float64) @ qr[0, h, 0].astype(np.float64) * scale
            p = np.exp(s - s.max())
            l = p.sum()
            v = vd[b, kh, :n].astype(np.float64)
            wabs[b, h] = (p[:, None] * np.abs(v)).sum(0) / l
            if case.quant == S.KV_INT8:
                nt = (n + 63) // 64
                w = np.zeros(nt * 64)
                w[:n] = p * oc.v_scale[b, kh, :n]
                c = np.zeros((nt * 64, D))
                c[:n] = np.abs(oc.v_codes[b, kh, :n].astype(np.float64))
                wmax = w.reshape(nt, 64).max(1)
                rep[b, h] = (wmax[:, None] * c.reshape(nt, 64, D).sum(1)).sum(0) / (64516.0 * l)
            else:
                z = oc.v_sz[b, kh, :n, :, 1].view(np.float16).astype(np.float64)  # [n, D/32]
                z = np.repeat(z, 32, axis=1)
                rep[b, h] = 2.0 ** -11 * (p[:, None] * np.abs(v - z)).sum(0) / l
    return wabs.reshape(B, 1, Hq * D), rep.reshape(B, 1, Hq * D)


def assert_close_decode_bound(got, ref, wabs, rep, what=""):
    """|got - ref| <= ATOL + RTOL |ref| + 2 (rep + 7e-5 sum p|v| / sum p): the
    kernel's weight representation (decode_weight_bounds) plus the oracle's
    expf_approx (3.5e-5 relative per weight, twice for the normalisation),
    with a factor 2 to spare."""
    err = np.abs(got - ref)
    tol = ATOL + RTOL * np.abs(ref) + 2.0 * (rep + 7e-5 * wabs)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside the bound; worst at {i}: got "
            f"{got[i]}, ref {ref[i]}, sum p|v| {wabs[i]:.4g}, weight bound {rep[i]:.4g}")
    return float((err / tol).max())
