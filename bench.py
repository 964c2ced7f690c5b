"""Benchmark of the compressed-KV GQA decode step on one MI355X.

Workload (the Llama-3-8B layer decode the metric is quoted on): 16 sequences,
32 query / 8 kv heads, head_dim 128, uniform context 8192 (8191 cached tokens
+ the step's token), Q bf16 ~ N(0,1), pre-RoPE K and V ~ N(0,1), RoPE theta
500000, int8 KV with one f32 scale per (token, kv head), 16-token pages.

One step = kernel 1 (RoPE + quantise + append the step's token for all 16x8
(sequence, kv head) rows) + kernel 2 (split-K flash decode over the 8192
tokens), i.e. one layer's attention for one generated token. The step's token
goes to the same slot every step (append without advance), so the context
stays at 8192.

Printed (one JSON line): whole-step algorithmic HBM throughput of the decode
attention (GB/s, `value`), % of the 8 TB/s peak, tokens/s, the decode
kernel's own roofline from HIP events on its stream, and the oracle (the C
restatement of the reference's single-threaded CPU path) timed on a bounded
sample on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode attention HBM GB/s (% of peak) + tokens/s, 8k ctx int8 KV, 1 MI355X"
PEAK_GBPS = 8000.0
B, HQ, HKV, D, CTX, THETA = 16, 32, 8, 128, 8192, 500000.0
PAGE = 16


def algorithmic_bytes(b=B, hq=HQ, hkv=HKV, d=D, ctx=CTX):
    """Bytes one decode step must move at minimum: int8 K+V codes, f32 K+V
    scales, the bf16 query and the f32 output."""
    codes = b * hkv * ctx * 2 * d
    scales = b * hkv * ctx * 2 * 4
    q = b * hq * d * 2
    out = b * hq * d * 4
    return codes + scales + q + out


def traffic_from_profile():
    """HBM bytes per decode launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, calibrated against a copy kernel), if the summary is present."""
    path = os.path.join(ROOT, "profiles", "gqa_decode_llama8k_pmc.txt")
    try:
        with open(path) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read(), re.M)
        return float(m.group(1)) if m else None
    except OSError:
        return None


def build_cache(S, torch, rt, cos_d, sin_d):
    pages = (CTX + PAGE - 1) // PAGE
    cache = S.KvCache(rt, 1, HKV, D, B * pages, B, pages, S.KV_INT8)
    cache.set_page_table(S.identity_page_table(B, pages))
    g = torch.Generator(device="cuda")
    g.manual_seed(0x5A1A0001)
    past = CTX - 1
    chunk = 1024
    done = 0
    while done < past:
        n = min(chunk, past - done)
        k = torch.randn((B, n, HKV * D), generator=g, device="cuda", dtype=torch.float32)
        v = torch.randn((B, n, HKV * D), generator=g, device="cuda", dtype=torch.float32)
        cache.append(0, k, v, B, n, cos_d, sin_d, cos_d.shape[0])
        cache.advance()
        done += n
    torch.cuda.synchronize()
    return cache, g


def copy_bandwidth(torch):
    """Device-to-device copy of 2 GiB: read + write bytes / time (a STREAM-like
    reference point for the 8 TB/s spec value)."""
    n = 1 << 29
    a = torch.empty(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1.0)
    for _ in range(3):
        b.copy_(a)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    reps = 10
    for _ in range(reps):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    del a, b
    return 2 * n * 4 / (ms * 1e-3) / 1e9


def cpu_baseline(seconds_target=12.0):
    """The oracle (C restatement of the reference's CPU path, one thread) on a
    bounded sample of the same workload: for each sampled sequence, quantise
    the appended token, dequantise its 8192-token int8 cache, RoPE Q, copy the
    present K/V and run the scalar f32 SDPA with expf_approx."""
    import oracle as O
    import smallaios_amd as S
    rng = np.random.default_rng(7)
    cos, sin = S.rope_tables(CTX, D, THETA)
    oc = O.LogicalCache(1, HKV, D, CTX, O.INT8)
    oc.k_codes[:] = rng.integers(-127, 128, oc.k_codes.shape, dtype=np.int8)
    oc.v_codes[:] = rng.integers(-127, 128, oc.v_codes.shape, dtype=np.int8)
    oc.k_scale[:] = rng.uniform(0.015, 0.035, oc.k_scale.shape).astype(np.float32)
    oc.v_scale[:] = rng.uniform(0.015, 0.035, oc.v_scale.shape).astype(np.float32)
    seqs = 0
    t0 = time.perf_counter()
    while True:
        oc.seq_len[:] = CTX - 1
        k = rng.standard_normal((1, 1, HKV * D), dtype=np.float32)
        v = rng.standard_normal((1, 1, HKV * D), dtype=np.float32)
        q = O.bf16_bits_to_f32(O.f32_to_bf16_bits(
            rng.standard_normal(HQ * D, dtype=np.float32))).reshape(1, 1, HQ * D)
        oc.append(k, v, cos, sin)
        oc.attend(q, HQ, cos, sin)
        seqs += 1
        el = time.perf_counter() - t0
        if el >= seconds_target and seqs % B == 0:
            break
    per_seq = el / seqs
    step_s = per_seq * B
    return {
        "value": round(algorithmic_bytes() / step_s / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{seqs} sequences ({seqs // B} full steps of {B}) of the 8192-context "
                   f"32Q/8KV int8 decode, one thread: {step_s * 1e3:.0f} ms per step, "
                   f"{B / step_s:.2f} tokens/s"),
        "ms_per_step": round(step_s * 1e3, 2),
        "tokens_per_s": round(B / step_s, 3),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--split", type=int, default=0, help="decode split size (0 = automatic)")
    ap.add_argument("--waves", type=int, default=0, help="waves per decode workgroup (4 or 8)")
    ap.add_argument("--unfused", action="store_true",
                    help="two launches per step (sai_kv_append + sai_gqa_decode) instead of the "
                         "fused sai_gqa_with_cache")
    ap.add_argument("--graph", action="store_true",
                    help="replay the step from a captured HIP graph (one graph launch per step)")
    ap.add_argument("--merge", choices=["auto", "combine", "inkernel"], default="auto",
                    help="split merge: separate combine kernel or last-workgroup merge")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this path is "
              "built and measured on a single MI355X. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import smallaios_amd as S

    assert torch.cuda.is_available(), "needs an MI355X"
    torch.cuda.set_device(0)
    rt = S.Runtime(0)
    if args.split:
        rt.set_decode_split(args.split)
    if args.waves:
        rt.set_decode_waves(args.waves)
    if args.merge != "auto":
        rt.set_decode_merge(args.merge == "inkernel")
    cos, sin = S.rope_tables(CTX, D, THETA)
    cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    cache, g = build_cache(S, torch, rt, cos_d, sin_d)

    q = torch.randn((B, 1, HQ * D), generator=g, device="cuda").to(torch.bfloat16)
    k_new = torch.randn((B, 1, HKV * D), generator=g, device="cuda")
    v_new = torch.randn((B, 1, HKV * D), generator=g, device="cuda")
    out = torch.empty((B, 1, HQ * D), device="cuda", dtype=torch.float32)
    stream = torch.cuda.Stream()  # default priority; graph capture needs a non-default stream
    rows = cos_d.shape[0]

    def step(ev=None):
        if args.unfused:
            cache.append(0, k_new, v_new, B, 1, cos_d, sin_d, rows, stream=stream)
        if ev is not None:
            ev[0].record(stream)
        if args.unfused:
            cache.decode(0, q, out, B, HQ, cos_d, sin_d, rows, stream=stream)
        else:
            cache.decode_with_cache(0, q, k_new, v_new, out, B, HQ, cos_d, sin_d, rows,
                                    stream=stream)
        if ev is not None:
            ev[1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    run = step
    if args.graph:
        # the step's launches (no allocation, no memset) recorded once, replayed
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            step()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        run = graph.replay

    # timed region 1: whole steps, wall clock
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall / args.steps * 1e3

    # timed region 2: the decode kernel alone, HIP events on its stream
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    kms = np.array([a.elapsed_time(b) for a, b in evs])
    k_us = float(np.median(kms)) * 1e3
    k_mean_us = float(kms.mean()) * 1e3
    wg, split = rt.last_decode_shape()

    alg = algorithmic_bytes()
    value = alg / (ms_step * 1e-3) / 1e9
    achieved = alg / (k_us * 1e-6) / 1e9
    copy_gbps = copy_bandwidth(torch)
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) Q/K/V, random-init; no checkpoint)",
        "config": {"workload": "llama3-8b-layer-gqa-decode", "batch": B, "context": CTX,
                   "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "q_dtype": "bf16",
                   "kv_cache": "int8 per-token-head f32 scale, 16-token pages",
                   "rope_theta": THETA,
                   "step": ("kv_append + gqa_decode" if args.unfused
                            else "gqa_with_cache (append fused into decode)")
                           + (", hip graph replay" if args.graph else "")},
        "pct_of_peak": round(100 * value / PEAK_GBPS, 2),
        "tokens_per_s": round(B / (ms_step * 1e-3), 1),
        "tokens_per_s_32_layers": round(B / (32 * ms_step * 1e-3), 1),
        "algorithmic_bytes_per_step": alg,
        "decode_kernel": {"median_us": round(k_us, 3), "mean_us": round(k_mean_us, 3),
                          "workgroups": wg, "split_tokens": split},
        "measured_copy_gbps": round(copy_gbps, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4),
                     "traffic": traffic_from_profile()},
    }
    cache.close()
    rt.close()
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
