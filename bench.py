"""Benchmark of the compressed-KV GQA path on one MI355X.

Default workload (the one the headline metric is quoted on): Llama-3-8B layer
decode -- 16 sequences, 32 query / 8 kv heads, head_dim 128, uniform context
8192 (8191 cached tokens + the step's token), Q bf16 ~ N(0,1), pre-RoPE K and
V ~ N(0,1), RoPE theta 500000, int8 KV with one f32 scale per (token, kv
head), 16-token pages.

One decode step = one layer's attention for one generated token per
sequence: RoPE + quantise + append the step's K/V and split-K flash decode
over the whole context (sai_gqa_with_cache: one decode launch that also
appends, plus the split-merge kernel). The step's token goes to the same slot
every step (append without advance), so the context stays fixed.

Other workloads (--workload, for the per-configuration table): `batch1`
(8Q/2KV, head_dim 64, context 512), `int4long` (4 sequences of 32768 tokens,
int4 KV with f16 (scale, zero) per group of 32 dims, K Student-t df 3 with
four x20 outlier channels), `gemma4b` and `gemma4b_int4` (Gemma 3 4B's 8Q/4KV at
head_dim 256, 16 sequences of 8192 tokens, int8 and int4 KV), `gemma31b` (Gemma 4
31B's 32Q/8KV at head_dim 168, stored 192 wide, 16 x 8192, int8), `ragged` (64 sequences with seeded lengths
U[128, 16384], randomly permuted page table), `prefill` (2 x 2048 new
tokens appended to a 6144-token cache, then causal MFMA attention) and `rope`
(the standalone RotaryEmbedding op over that chunk's queries: [2, 2048,
32*128] bf16 in the [B, S, H*D] layout at positions 6144.., out of place,
f32 tables; an f32 input is timed beside it).

Printed: one JSON line with whole-step algorithmic throughput (`value`), % of
peak, tokens/s, the dominant kernel's roofline from HIP events on its stream,
and (default workload) the oracle -- the C restatement of the reference's
single-threaded CPU path -- timed on a bounded sample on the host cores.
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
HBM_PEAK_GBPS = 8000.0       # MI355X HBM3E spec
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16/bf16 matrix peak
PAGE = 16

WORKLOADS = {
    "llama8k": dict(kind="decode", batch=16, hq=32, hkv=8, d=128, lens=("uniform", 8192),
                    theta=500000.0, q_dtype="bf16", permute=False),
    "batch1": dict(kind="decode", batch=1, hq=8, hkv=2, d=64, lens=("uniform", 512),
                   theta=10000.0, q_dtype="f32", permute=False),
    "int4long": dict(kind="decode", batch=4, hq=32, hkv=8, d=128, lens=("uniform", 32768),
                     theta=500000.0, q_dtype="bf16", permute=False, quant="int4",
                     k_dist="outlier_t3"),
    "gemma4b": dict(kind="decode", batch=16, hq=8, hkv=4, d=256, lens=("uniform", 8192),
                    theta=1000000.0, q_dtype="bf16", permute=False),
    "gemma4b_int4": dict(kind="decode", batch=16, hq=8, hkv=4, d=256, lens=("uniform", 8192),
                         theta=1000000.0, q_dtype="bf16", permute=False, quant="int4",
                         k_dist="outlier_t3"),
    "gemma31b": dict(kind="decode", batch=16, hq=32, hkv=8, d=168, lens=("uniform", 8192),
                     theta=1000000.0, q_dtype="bf16", permute=False),
    "ragged": dict(kind="decode", batch=64, hq=32, hkv=8, d=128, lens=("uniform_rand", 128, 16384),
                   theta=500000.0, q_dtype="bf16", permute=True),
    "prefill": dict(kind="prefill", batch=2, hq=32, hkv=8, d=128, past=6144, new=2048,
                    theta=500000.0, q_dtype="bf16", permute=False),
    "rope": dict(kind="rotary", batch=2, hq=32, d=128, past=6144, new=2048, theta=500000.0),
    "tq4": dict(kind="tq", batch=16, hq=32, hkv=8, d=128, ctx=8192, bits=4, qjl=True,
                q_dtype="bf16"),
}


def tq_bytes_per_row_head(d, bits, qjl):
    """What TurboQuant decode attention must read per (row, kv head): K and V
    codes, K (scale, zero[, QJL mean]), V (scale, zero), K's QJL sign bits."""
    return 2 * d * bits // 8 + (12 if qjl else 8) + 8 + (d // 8 if qjl else 0)


def decode_lengths(w, seed=0x5A1A0003):
    kind = w["lens"][0]
    if kind == "uniform":
        return np.full(w["batch"], w["lens"][1], dtype=np.int64)
    rng = np.random.default_rng(seed)
    return rng.integers(w["lens"][1], w["lens"][2] + 1, size=w["batch"]).astype(np.int64)


def stored_dim(d):
    """Row width the cache stores: head_dim 168 is kept 192 wide (each 84-dim
    half of the split-half RoPE pairing followed by 12 zero dims)."""
    return 192 if d == 168 else d


def kv_bytes_per_token_head(d, quant, stored=True):
    """int8: K+V codes (2d) and two f32 scales; int4: K+V nibbles (d) and an
    f16 (scale, zero) per group of 32 dims for K and for V (d/4). d is the
    stored width unless `stored` is False (the caller's head_dim)."""
    d = stored_dim(d) if stored else d
    return 2 * d + 8 if quant == "int8" else d + d // 4


def decode_bytes(lens, hq, hkv, d, q_bytes, quant="int8", stored=True):
    """Algorithmic bytes of one decode step: the K+V codes and quantisation
    parameters of every visible token (at the stored row width, or the
    caller's head_dim when `stored` is False), the query and the f32 output."""
    kv = int(lens.sum()) * hkv * kv_bytes_per_token_head(d, quant, stored)
    return kv + len(lens) * hq * d * q_bytes + len(lens) * hq * d * 4


def prefill_flops(batch, hq, d, past, new):
    """QK^T + PV multiply-adds x2 over every (query, visible key) pair."""
    keys = sum(past + i + 1 for i in range(new))
    return 4 * d * hq * keys * batch


def append_roofline(b, new, hkv, d, us):
    """HBM roofline of the int8 append of `new` bf16 tokens per sequence:
    K and V rows read (2 bytes an element), codes and two f32 scales per
    (token, kv head) written, and one cos and one sin row of D/2 f32 per
    position read."""
    rows = b * new * hkv
    alg = rows * d * 2 * 2 + rows * (2 * d + 8) + b * new * d * 4
    gbps = alg / (us * 1e-6) / 1e9
    return {"median_us": round(us, 2), "algorithmic_bytes": alg, "achieved_gbps": round(gbps, 1),
            "peak_gbps": HBM_PEAK_GBPS, "frac": round(gbps / HBM_PEAK_GBPS, 4)}


def traffic_from_profile(workload, kernel="gqa_decode"):
    """HBM bytes per launch of the workload's dominant kernel measured with
    rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, calibrated against a copy of
    known size), if the workload's summary is present."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_pmc.txt")
    try:
        with open(path) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read(), re.M)
        return float(m.group(1)) if m else None
    except OSError:
        return None


def build_cache(S, torch, rt, w, past_lens, extra_tokens, cos_d, sin_d, seed):
    """Cache holding past_lens[b] tokens per sequence, appended by the HIP
    append kernel in chunks (all sequences to max(past), then truncated)."""
    b, hkv, d = w["batch"], w["hkv"], w["d"]
    cap = int(past_lens.max()) + extra_tokens
    pages = (cap + PAGE - 1) // PAGE
    quant = S.KV_INT4 if w.get("quant") == "int4" else S.KV_INT8
    cache = S.KvCache(rt, 1, hkv, d, b * pages, b, pages, quant)
    ids = np.arange(b * pages, dtype=np.int32)
    if w["permute"]:
        ids = np.random.default_rng(seed).permutation(ids).astype(np.int32)
    cache.set_page_table(ids.reshape(b, pages))
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    # chunks of ~131k (token, kv head) rows per append call, the Llama-3-8B
    # layer's 16 x 1024 (at least 1024 tokens)
    chunk = max(1024, (131072 // (b * hkv)) // PAGE * PAGE)
    past, done = int(past_lens.max()), 0
    while done < past:
        n = min(chunk, past - done)
        k = torch.randn((b, n, hkv * d), generator=g, device="cuda")
        v = torch.randn((b, n, hkv * d), generator=g, device="cuda")
        if w.get("k_dist") == "outlier_t3":
            # Student-t df 3 (normal / sqrt(chi2_3 / 3)), four x20 channels per head
            chi = torch.randn((3, b, n, hkv * d), generator=g, device="cuda").square().sum(0)
            k = (k / torch.sqrt(chi / 3)).view(b, n, hkv, d)
            k[..., [7, 31, 64, 100]] *= 20.0
            k = k.reshape(b, n, hkv * d).contiguous()
        cache.append(0, k, v, b, n, cos_d, sin_d, cos_d.shape[0])
        cache.advance()
        done += n
    cache.set_seq_lens(past_lens.astype(np.int32))
    torch.cuda.synchronize()
    return cache, g


INFINITY_CACHE_BYTES = 256 << 20  # MI355X last-level (Infinity) cache


def split_balance(lens, split, hkv, slots=512):
    """Load balance of the split-K partition of a ragged batch: the tokens of
    each (sequence, split) workgroup, their spread, and a list-scheduling
    model of the launch (workgroups taken in launch order by the first free
    of `slots` workgroup slots -- 256 CUs x 2 four-wave workgroups -- each
    busy for its token count) against the perfectly balanced time
    sum(tokens) / slots. A model of the dispatch, not a measurement."""
    import heapq
    toks = []
    for L in lens:
        L = int(L)
        n = (L + split - 1) // split
        toks += [min(split, L - i * split) for i in range(n)]
    # grid x = (sequence, split) items, y = kv heads: dispatched x fastest
    per_wg = np.tile(np.array(toks, dtype=np.int64), hkv)
    free = [0] * slots
    for t in per_wg:
        heapq.heapreplace(free, free[0] + int(t))
    ideal = per_wg.sum() / slots
    return {"splits": len(toks), "workgroups": int(per_wg.size),
            "tokens_per_split": {"min": int(min(toks)), "mean": round(float(np.mean(toks)), 1),
                                 "max": int(max(toks))},
            "mean_over_max": round(float(np.mean(toks)) / max(toks), 4),
            "list_schedule_makespan_over_ideal": round(float(max(free) / ideal), 4),
            "model": f"{slots} workgroup slots, duration proportional to tokens"}


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


def read_ceiling(torch, nbytes):
    """The best streaming-read rate of a plain kernel (16-byte non-temporal
    loads, one contiguous slice per workgroup) over `nbytes` of device memory,
    swept over the workgroup count: an achievable ceiling measured in the same
    run, beside the 8 TB/s spec value."""
    import ctypes as C
    here = os.path.dirname(os.path.abspath(__file__))
    lib = C.CDLL(os.path.join(here, "smallaios_amd", "libsai_read_probe.so"))
    lib.sai_probe_stream_read.restype = C.c_int
    lib.sai_probe_stream_read.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int,
                                          C.c_void_p, C.c_void_p, C.POINTER(C.c_float)]
    nbytes -= nbytes % 16
    buf = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
    best = {}
    sweep = {}
    stream = torch.cuda.current_stream().cuda_stream
    for wgs in (256, 512, 1024, 2048, 4096, 8192):
        sink = torch.zeros(wgs, dtype=torch.int32, device="cuda")
        us = C.c_float(0.0)
        rc = lib.sai_probe_stream_read(buf.data_ptr(), nbytes, wgs, 10, 100, sink.data_ptr(),
                                       stream, C.byref(us))
        if rc != 0:
            raise RuntimeError(f"read probe failed: hipError {rc}")
        gbps = nbytes / (us.value * 1e-6) / 1e9
        sweep[str(wgs)] = round(gbps, 1)
        if gbps > best.get("gbps", 0.0):
            best = {"gbps": round(gbps, 1), "workgroups": wgs, "us": round(us.value, 2)}
    del buf
    best["sweep_gbps_by_workgroups"] = sweep
    return best


def cpu_baseline(w, seconds_target=12.0):
    """The oracle (C restatement of the reference's CPU path, one thread) on a
    bounded sample of the default workload: per sampled sequence, quantise the
    appended token, dequantise its int8 cache, RoPE Q, copy the present K/V and
    run the scalar f32 SDPA with expf_approx."""
    import oracle as O
    import smallaios_amd as S
    hq, hkv, d, ctx, theta = w["hq"], w["hkv"], w["d"], w["lens"][1], w["theta"]
    rng = np.random.default_rng(7)
    cos, sin = S.rope_tables(ctx, d, theta)
    oc = O.LogicalCache(1, hkv, d, ctx, O.INT8)
    oc.k_codes[:] = rng.integers(-127, 128, oc.k_codes.shape, dtype=np.int8)
    oc.v_codes[:] = rng.integers(-127, 128, oc.v_codes.shape, dtype=np.int8)
    oc.k_scale[:] = rng.uniform(0.015, 0.035, oc.k_scale.shape).astype(np.float32)
    oc.v_scale[:] = rng.uniform(0.015, 0.035, oc.v_scale.shape).astype(np.float32)
    seqs = 0
    t0 = time.perf_counter()
    while True:
        oc.seq_len[:] = ctx - 1
        k = rng.standard_normal((1, 1, hkv * d), dtype=np.float32)
        v = rng.standard_normal((1, 1, hkv * d), dtype=np.float32)
        q = O.bf16_bits_to_f32(O.f32_to_bf16_bits(
            rng.standard_normal(hq * d, dtype=np.float32))).reshape(1, 1, hq * d)
        oc.append(k, v, cos, sin)
        oc.attend(q, hq, cos, sin)
        seqs += 1
        el = time.perf_counter() - t0
        if el >= seconds_target and seqs % w["batch"] == 0:
            break
    step_s = el / seqs * w["batch"]
    lens = decode_lengths(w)
    return {
        "value": round(decode_bytes(lens, hq, hkv, d, 2) / step_s / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{seqs} sequences ({seqs // w['batch']} full steps of {w['batch']}) of the "
                   f"{ctx}-context {hq}Q/{hkv}KV int8 decode, one thread: "
                   f"{step_s * 1e3:.0f} ms per step, {w['batch'] / step_s:.2f} tokens/s"),
        "ms_per_step": round(step_s * 1e3, 2),
        "tokens_per_s": round(w["batch"] / step_s, 3),
        "threads": 1,
        "host_nproc": os.cpu_count(),
        "host_cpus_usable": len(os.sched_getaffinity(0)),
        "host_cpu": host_cpu_model(),
    }


def host_cpu_model():
    """The CPU model string of /proc/cpuinfo (None where there is none)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def settle(torch, run, seconds):
    """Untimed: runs the step until `seconds` of wall time have passed, so that
    the GPU's clocks are at their steady state under this load before the
    warmup and the timed steps. Measured at the Llama-3-8B decode shape: after
    50 warmup steps alone the timed steps ran 2.5-3.5 % slower than after
    250 ms of steps."""
    if seconds <= 0:
        return
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            run()
        torch.cuda.synchronize()


def time_steps(torch, run, steps):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


def kernel_times(torch, rt, pre, kernel, steps):
    """Decode-kernel duration of each launch from the HIP events the library
    records on the launch stream around that kernel alone (not the split
    merge that follows it); launches run back to back, as in the timed loop."""
    n = min(steps, 4096)
    rt.set_decode_timing(n)
    try:
        for _ in range(n):
            pre()
            kernel()
        out = rt.decode_kernel_times(n)
    finally:
        rt.set_decode_timing(0)
    return np.array(out)


def event_times(torch, stream, pre, kernel, steps):
    """Per-launch duration of `kernel` from HIP events recorded on its stream
    around it (the rest of the step, `pre`, runs outside the bracket)."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for a, b in evs:
        pre()
        a.record(stream)
        kernel()
        b.record(stream)
    torch.cuda.synchronize()
    return np.array([a.elapsed_time(b) for a, b in evs]) * 1e3  # us


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="llama8k")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--settle", type=float, default=0.25,
                    help="seconds of untimed steps before the warmup (clocks to steady state)")
    ap.add_argument("--split", type=int, default=0, help="decode split size (0 = automatic)")
    ap.add_argument("--waves", type=int, default=0, help="waves per decode workgroup (4 or 8)")
    ap.add_argument("--unfused", action="store_true",
                    help="decode: sai_kv_append + sai_gqa_decode instead of sai_gqa_with_cache")
    ap.add_argument("--tile-order", choices=["auto", "fixed", "dynamic"], default="auto",
                    help="int8 decode tile order (fixed: bit-reproducible outputs)")
    ap.add_argument("--merge", choices=["auto", "combine", "inkernel"], default="auto",
                    help="decode split merge: combine kernel or last-workgroup merge")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this path is "
              "built and measured on a single MI355X. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import smallaios_amd as S

    assert torch.cuda.is_available(), "needs an MI355X"
    torch.cuda.set_device(0)
    w = WORKLOADS[args.workload]
    rt = S.Runtime(0)
    if args.split:
        rt.set_decode_split(args.split)
        rt.set_tq_split(args.split)
    if args.waves:
        rt.set_decode_waves(args.waves)
    if args.merge != "auto":
        rt.set_decode_merge(1 if args.merge == "inkernel" else 0)
    if args.tile_order != "auto":
        rt.set_decode_reproducible(1 if args.tile_order == "fixed" else 0)
    b, hq, hkv, d = w["batch"], w["hq"], w.get("hkv", 0), w["d"]
    qdt = torch.bfloat16 if w.get("q_dtype", "bf16") == "bf16" else torch.float32
    stream = torch.cuda.Stream()  # default priority
    seed = 0x5A1A0001

    if w["kind"] == "decode":
        lens = decode_lengths(w)
        cos, sin = S.rope_tables(int(lens.max()) + 1, d, w["theta"])
        cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
        cache, g = build_cache(S, torch, rt, w, lens - 1, 1, cos_d, sin_d, seed)
        q = torch.randn((b, 1, hq * d), generator=g, device="cuda").to(qdt)
        k_new = torch.randn((b, 1, hkv * d), generator=g, device="cuda")
        v_new = torch.randn((b, 1, hkv * d), generator=g, device="cuda")
        out = torch.empty((b, 1, hq * d), device="cuda", dtype=torch.float32)
        rows = cos_d.shape[0]

        def pre():
            if args.unfused:
                cache.append(0, k_new, v_new, b, 1, cos_d, sin_d, rows, stream=stream)

        def kern():
            if args.unfused:
                cache.decode(0, q, out, b, hq, cos_d, sin_d, rows, stream=stream)
            else:
                cache.decode_with_cache(0, q, k_new, v_new, out, b, hq, cos_d, sin_d, rows,
                                        stream=stream)

        def step():
            pre()
            kern()

        settle(torch, step, args.settle)
        for _ in range(args.warmup):
            step()
        ms_step = time_steps(torch, step, args.steps)
        kus = event_times(torch, stream, pre, kern, args.steps)  # decode + merge
        dus = kernel_times(torch, rt, pre, kern, args.steps)     # decode kernel alone
        wg, split = rt.last_decode_shape()
        quant = w.get("quant", "int8")
        alg = decode_bytes(lens, hq, hkv, d, 2 if qdt == torch.bfloat16 else 4, quant)
        rotated = None
        if alg < INFINITY_CACHE_BYTES:
            # the step's bytes fit in the 256 MB Infinity Cache: time it again
            # alternating between two caches of the same shape (different
            # contents), so every step's stream comes from HBM
            cache2, _ = build_cache(S, torch, rt, w, lens - 1, 1, cos_d, sin_d, seed + 1)
            caches = (cache, cache2)
            flip = [0]

            def step2():
                c = caches[flip[0]]
                flip[0] ^= 1
                if args.unfused:
                    c.append(0, k_new, v_new, b, 1, cos_d, sin_d, rows, stream=stream)
                    c.decode(0, q, out, b, hq, cos_d, sin_d, rows, stream=stream)
                else:
                    c.decode_with_cache(0, q, k_new, v_new, out, b, hq, cos_d, sin_d, rows,
                                        stream=stream)

            for _ in range(args.warmup):
                step2()
            ms2 = time_steps(torch, step2, args.steps)
            cache2.close()
            v2 = alg / (ms2 * 1e-3) / 1e9
            rotated = {"ms_per_step": round(ms2, 5), "value": round(v2, 1),
                       "pct_of_peak": round(100 * v2 / HBM_PEAK_GBPS, 2),
                       "working_set_bytes": 2 * alg,
                       "note": "steps alternate between two caches (2x the step's bytes, "
                               "above the 256 MB Infinity Cache)"}
        k_us = float(np.median(kus))
        d_us = float(np.mean(dus))
        value = alg / (ms_step * 1e-3) / 1e9
        # one launch per step (the fused step merging its splits in-kernel):
        # the step clock, over back-to-back launches, prices the decode kernel
        # itself; HIP events around single launches add dispatch latency.
        # Otherwise (a combine kernel or a separate append follows or precedes
        # it) the events around the decode kernel alone.
        single_launch = not args.unfused and rt.last_decode_launches() == 1
        kernel_us = ms_step * 1e3 if single_launch else d_us
        # a step that fits the Infinity Cache is priced on the loop that
        # alternates two caches, so the roofline is that of the HBM stream
        hbm_clock = single_launch and rotated is not None
        if hbm_clock:
            kernel_us = rotated["ms_per_step"] * 1e3
        achieved = alg / (kernel_us * 1e-6) / 1e9
        result = {
            "metric": METRIC if args.workload == "llama8k" else
            f"{args.workload} decode attention HBM GB/s, {quant} KV, 1 MI355X",
            "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "settle_s": args.settle, "ms_per_step": round(ms_step, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None,
            "dtype": "int8" if quant == "int8" else "int8 QK / f16 PV",
            "data": ("synthetic (seeded N(0,1) Q/V, K "
                     + ("Student-t df 3 with x20 outlier channels" if w.get("k_dist") else "N(0,1)")
                     + "; no checkpoint)"),
            "config": {"workload": args.workload, "batch": b, "q_heads": hq, "kv_heads": hkv,
                       "head_dim": d, "context": (int(lens[0]) if w["lens"][0] == "uniform"
                                                  else f"U[{w['lens'][1]},{w['lens'][2]}]"),
                       "total_tokens": int(lens.sum()), "q_dtype": w["q_dtype"],
                       "kv_cache": ("int8 per-token-head f32 scale" if quant == "int8" else
                                    "int4 asymmetric, f16 (scale, zero) per group of 32 dims")
                                   + ", 16-token pages"
                                   + (", permuted page table" if w["permute"] else ""),
                       "rope_theta": w["theta"],
                       "step": ("kv_append + gqa_decode (+ merge)" if args.unfused
                                else "gqa_with_cache: append fused into decode (+ merge)")},
            "pct_of_peak": round(100 * value / HBM_PEAK_GBPS, 2),
            "tokens_per_s": round(b / (ms_step * 1e-3), 1),
            "tokens_per_s_32_layers": round(b / (32 * ms_step * 1e-3), 1),
            "algorithmic_bytes_per_step": alg,
            "decode_kernel": {"mean_us": round(d_us, 3), "median_us": round(float(np.median(dus)), 3),
                              "workgroups": wg, "split_tokens": split},
            "decode_plus_merge_us": {"median": round(k_us, 3), "mean": round(float(kus.mean()), 3)},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                         "traffic": traffic_from_profile(args.workload),
                         "kernel_us": round(kernel_us, 3),
                         "basis": ("step clock over back-to-back steps of one decode launch "
                                   "each, alternating two caches so the stream comes from HBM"
                                   if hbm_clock else
                                   "step clock over back-to-back steps of one decode launch "
                                   "each (the fused step, splits merged in-kernel)"
                                   if single_launch else
                                   "mean of HIP events recorded on the launch stream around "
                                   "each decode launch (they include a few us of dispatch "
                                   "latency)")},
        }
        if rotated is not None:
            result["rotated_two_caches"] = rotated
        if stored_dim(d) != d:
            # the caller's bytes (168-dim rows) moved per second: the padding
            # of the stored rows is traffic this layout adds
            lg = decode_bytes(lens, hq, hkv, d, 2 if qdt == torch.bfloat16 else 4, quant,
                              stored=False)
            result["stored_head_dim"] = stored_dim(d)
            result["logical_bytes_per_step"] = lg
            result["logical_gbps"] = round(lg / (ms_step * 1e-3) / 1e9, 1)
        if w["lens"][0] != "uniform":
            result["split_balance"] = split_balance(lens, split, hkv)
    elif w["kind"] == "rotary":
        past, new = w["past"], w["new"]
        half = d // 2
        cos, sin = S.rope_tables(past + new, d, w["theta"])
        cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        runs = {}
        for name, dt in (("bf16", torch.bfloat16), ("f32", torch.float32)):
            x = torch.randn((b, new, hq * d), generator=g, device="cuda").to(dt)
            y = torch.empty_like(x)

            def kern(x=x, y=y):
                rt.rotary_embedding(x, y, b, hq, new, d, cos_d, sin_d, start_position=past,
                                    layout=S.ROPE_BSHD, stream=stream)

            settle(torch, kern, args.settle)
            for _ in range(args.warmup):
                kern()
            ms = time_steps(torch, kern, args.steps)
            kus = event_times(torch, stream, lambda: None, kern, args.steps)
            # x read once, y written once, the chunk's table rows read once
            alg = 2 * x.numel() * x.element_size() + 2 * new * half * 4
            runs[name] = (ms, float(np.median(kus)), alg)
        ms_step, k_us, alg = runs["bf16"]
        achieved = alg / (k_us * 1e-6) / 1e9
        result = {
            "metric": "RotaryEmbedding HBM GB/s (% of peak), 1 MI355X",
            "value": round(alg / (ms_step * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "settle_s": args.settle, "ms_per_step": round(ms_step, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) queries; no checkpoint)",
            "config": {"workload": "rope", "batch": b, "heads": hq, "head_dim": d,
                       "seq": new, "start_position": past, "layout": "[B, S, H*D]",
                       "tables": "f32 [8192, 64]", "rope_theta": w["theta"]},
            "algorithmic_bytes_per_step": alg,
            "rotary_kernel": {"median_us": round(k_us, 3)},
            "f32_input": {"median_us": round(runs["f32"][1], 3),
                          "gbps": round(runs["f32"][2] / (runs["f32"][1] * 1e-6) / 1e9, 1)},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                         "traffic": None},
        }
        cache = None
    elif w["kind"] == "tq":
        ctx, bits, qjl = w["ctx"], w["bits"], w["qjl"]
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)

        def build_tq():
            c = S.TqCache(rt, 1, hkv, d, bits, qjl, b, ctx, seed=0x5EED)
            done = 0
            while done < ctx - 1:
                n = min(1024, ctx - 1 - done)
                k = torch.randn((b, n, hkv * d), generator=g, device="cuda")
                v = torch.randn((b, n, hkv * d), generator=g, device="cuda")
                c.write(0, k, v, b, n)
                c.advance()
                done += n
            torch.cuda.synchronize()
            return c

        cache = build_tq()
        q = torch.randn((b, 1, hq * d), generator=g, device="cuda").to(qdt)
        k_new = torch.randn((b, 1, hkv * d), generator=g, device="cuda").to(qdt)
        v_new = torch.randn((b, 1, hkv * d), generator=g, device="cuda").to(qdt)
        out = torch.empty((b, 1, hq * d), device="cuda", dtype=torch.float32)

        def pre():
            if args.unfused:
                cache.write(0, k_new, v_new, b, 1, stream=stream)

        def kern():
            if args.unfused:
                cache.attend(0, q, out, b, hq, stream=stream)
            else:
                cache.write_attend(0, q, k_new, v_new, out, b, hq, stream=stream)

        def step():
            pre()  # each step rewrites the pending row: every step sees ctx rows
            kern()

        settle(torch, step, args.settle)
        for _ in range(args.warmup):
            step()
        ms_step = time_steps(torch, step, args.steps)
        kus = event_times(torch, stream, pre, kern, args.steps)   # query + attend + merge
        wus = event_times(torch, stream, lambda: None,
                          lambda: cache.write(0, k_new, v_new, b, 1, stream=stream), args.steps)
        per = tq_bytes_per_row_head(d, bits, qjl)
        alg = b * ctx * hkv * per + b * hq * d * (2 + 4)
        rotated = None
        if alg < INFINITY_CACHE_BYTES:
            # as for the decode workloads: alternate two caches so the stream
            # cannot come from the 256 MB Infinity Cache
            cache2 = build_tq()
            caches = (cache, cache2)
            flip = [0]

            def step2():
                c = caches[flip[0]]
                flip[0] ^= 1
                if args.unfused:
                    c.write(0, k_new, v_new, b, 1, stream=stream)
                    c.attend(0, q, out, b, hq, stream=stream)
                else:
                    c.write_attend(0, q, k_new, v_new, out, b, hq, stream=stream)

            for _ in range(args.warmup):
                step2()
            ms2 = time_steps(torch, step2, args.steps)
            cache2.close()
            v2 = alg / (ms2 * 1e-3) / 1e9
            rotated = {"ms_per_step": round(ms2, 5), "value": round(v2, 1),
                       "pct_of_peak": round(100 * v2 / HBM_PEAK_GBPS, 2),
                       "working_set_bytes": 2 * alg,
                       "note": "steps alternate between two caches (2x the step's bytes, "
                               "above the 256 MB Infinity Cache)"}
        k_us = float(np.median(kus))
        # the fused step is one launch: with two caches alternating (the
        # stream from HBM, not the Infinity Cache) its step clock prices the
        # kernel; otherwise the events around each attention launch
        hbm_clock = not args.unfused and rotated is not None
        kernel_us = rotated["ms_per_step"] * 1e3 if hbm_clock else k_us
        achieved = alg / (kernel_us * 1e-6) / 1e9
        result = {
            "metric": "TurboQuant decode attention HBM GB/s (% of peak), 1 MI355X",
            "value": round(alg / (ms_step * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "settle_s": args.settle, "ms_per_step": round(ms_step, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32 on u%d codes" % bits,
            "data": "synthetic (seeded N(0,1) Q/K/V; no checkpoint)",
            "config": {"workload": "tq4", "batch": b, "q_heads": hq, "kv_heads": hkv,
                       "head_dim": d, "context": ctx, "bits": bits, "qjl": qjl,
                       "step": ("tq_cache_write (1 token, pending) + tq_cache_attend"
                                if args.unfused else
                                "tq_cache_write_attend: the token's store fused into the "
                                "attention kernel (+ split merge)")},
            "algorithmic_bytes_per_step": alg,
            "bytes_per_row_head": per,
            "attend_us": {"median": round(k_us, 3), "mean": round(float(kus.mean()), 3)},
            "separate_write_us": {"median": round(float(np.median(wus)), 3)},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                         "traffic": traffic_from_profile(args.workload, "tq_attend"),
                         "kernel_us": round(kernel_us, 3),
                         "basis": ("step clock over back-to-back steps of one launch each "
                                   "(query encoding + attention + split merge), alternating "
                                   "two caches so the stream comes from HBM" if hbm_clock else
                                   "median of HIP events around each attention launch "
                                   "(query encoding + attention + split merge)")},
        }
        if rotated is not None:
            result["rotated_two_caches"] = rotated
    else:  # prefill
        past, new = w["past"], w["new"]
        cos, sin = S.rope_tables(past + new, d, w["theta"])
        cos_d, sin_d = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
        cache, g = build_cache(S, torch, rt, w, np.full(b, past), new, cos_d, sin_d, seed)
        q = torch.randn((b, new, hq * d), generator=g, device="cuda").to(qdt)
        k_new = torch.randn((b, new, hkv * d), generator=g, device="cuda").to(torch.bfloat16)
        v_new = torch.randn((b, new, hkv * d), generator=g, device="cuda").to(torch.bfloat16)
        out = torch.empty((b, new, hq * d), device="cuda", dtype=torch.float32)
        rows = cos_d.shape[0]

        def pre():
            cache.append(0, k_new, v_new, b, new, cos_d, sin_d, rows, stream=stream)

        def kern():
            cache.prefill(0, q, out, b, new, hq, cos_d, sin_d, rows, stream=stream)

        def step():
            pre()
            kern()

        settle(torch, step, args.settle)
        for _ in range(args.warmup):
            step()
        ms_step = time_steps(torch, step, args.steps)
        kus = event_times(torch, stream, pre, kern, args.steps)
        aus = event_times(torch, stream, lambda: None, pre, max(10, args.steps // 4))
        flops = prefill_flops(b, hq, d, past, new)
        k_us = float(np.median(kus))
        tflops = flops / (k_us * 1e-6) / 1e12
        result = {
            "metric": "prefill chunk attention TFLOP/s (MFMA), int8 KV, 1 MI355X",
            "value": round(flops / (ms_step * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "settle_s": args.settle, "ms_per_step": round(ms_step, 5),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
            "data": "synthetic (seeded N(0,1) Q/K/V; no checkpoint)",
            "config": {"workload": "prefill", "batch": b, "q_heads": hq, "kv_heads": hkv,
                       "head_dim": d, "past": past, "new_tokens": new, "q_dtype": "bf16",
                       "kv_cache": "int8 per-token-head f32 scale, 16-token pages",
                       "step": "kv_append (2048 tokens) + gqa_prefill"},
            "tokens_per_s": round(b * new / (ms_step * 1e-3), 1),
            "prefill_kernel": {"median_us": round(k_us, 2), "flops": flops},
            "append_kernel": append_roofline(b, new, hkv, d, float(np.median(aus))),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                         "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None},
        }
    result["measured_copy_gbps"] = round(copy_bandwidth(torch), 1)
    if w["kind"] == "decode" and result["algorithmic_bytes_per_step"] >= 1 << 26:
        rc = read_ceiling(torch, result["algorithmic_bytes_per_step"])
        result["measured_read_ceiling"] = {
            **rc, "bytes": result["algorithmic_bytes_per_step"],
            "step_frac": round(result["value"] / rc["gbps"], 4),
            "decode_kernel_frac": round(result["roofline"]["achieved"] / rc["gbps"], 4)}
    if cache is not None:
        cache.close()
    rt.close()
    if args.workload == "llama8k" and not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(w)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
