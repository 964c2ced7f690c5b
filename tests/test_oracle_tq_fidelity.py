"""Fidelity of the TurboQuant cache against uncompressed attention, on the
oracle (CPU).

Restates the reference's integration_synthetic_gqa_compressed_vs_uncompressed
(onnx-rt/src/kv_compression.rs:1752-1829): 32 K/V rows of head_dim 64 drawn
from xorshift64 (seed 12345) as (next() as f32 / u64::MAX as f32) * 2 - 1,
written to a 4-bit + QJL cache (seed 42, one layer, one kv head), K read back
with read_k, and the logits of the raw query against read_k compared with the
uncompressed logits: max error / mean |logit| < 1.0.

The same bar is applied to the estimator the GPU attention evaluates (the
query quantised with the head's quantiser, the inner product of the two
decodes plus the QJL correction, docs/kv-compression-design.md section 9),
and the estimator is checked to be the same quantity as <decode(q), read_k>
up to the correction term.
"""
import numpy as np

import oracle as O

DIM, SEQ, BITS, SEED = 64, 32, 4, 42
M64 = (1 << 64) - 1


def xorshift64(seed):
    """Xorshift64 of the reference (kv_compression.rs:44-67)."""
    s = seed if seed != 0 else 0x5EEDDEADBEEFCAFE
    while True:
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        yield s


def u64_as_f32(x: int) -> np.float32:
    """Rust's `x as f32` for a u64: one rounding to nearest, ties to even."""
    n = x.bit_length()
    if n <= 24:
        return np.float32(x)
    shift = n - 24
    mant, rem, half = x >> shift, x & ((1 << shift) - 1), 1 << (shift - 1)
    if rem > half or (rem == half and (mant & 1)):
        mant += 1
    return np.float32(float(mant) * 2.0 ** shift)


def reference_rows():
    """all_k [32, 64], all_v [32, 64], query [64] as the reference draws them."""
    g = xorshift64(12345)
    umax = u64_as_f32(M64)
    one, two = np.float32(1.0), np.float32(2.0)

    def draw():
        return np.array([(u64_as_f32(next(g)) / umax) * two - one for _ in range(DIM)],
                        np.float32)

    ks, vs = [], []
    for _ in range(SEQ):
        ks.append(draw())
        vs.append(draw())
    return np.stack(ks), np.stack(vs), draw()


def test_u64_as_f32_rounding():
    assert u64_as_f32(M64) == np.float32(2.0 ** 64)
    assert u64_as_f32((1 << 24) + 1) == np.float32(1 << 24)        # tie -> even
    assert u64_as_f32((1 << 24) + 3) == np.float32((1 << 24) + 4)  # tie -> even (up)
    assert u64_as_f32((1 << 40) + (1 << 16) + 1) == np.float32((1 << 40) + (1 << 17))


def test_reference_compressed_vs_uncompressed_logits():
    k, v, q = reference_rows()
    assert np.all(np.abs(k) <= 1.0) and np.all(np.abs(q) <= 1.0)
    sg = O.tq_signs(O.tq_head_seed(SEED, 0, 1, 0), DIM)
    codes, sc, z, sb, c = O.tq_write_rows(k, BITS, sg, True)
    k_read = np.stack([O.tq_decode(codes[t], DIM, BITS, sc[t], z[t], sg) for t in range(SEQ)])
    true = k.astype(np.float64) @ q.astype(np.float64)
    comp = k_read.astype(np.float64) @ q.astype(np.float64)
    rel = np.abs(true - comp).max() / (np.abs(true).mean() + 1e-6)
    assert rel < 1.0, rel

    # the estimator of the decode path: the query encoded by the same
    # quantiser, <decode(q), read_k> plus the QJL correction
    logits = O.tq_attention_logits(q[None, :], BITS, True, sg, (codes, sc, z, sb, c))[0]
    rel_est = np.abs(true - logits).max() / (np.abs(true).mean() + 1e-6)
    assert rel_est < 1.0, rel_est
    qc, qs, qz, qsb, qcm = O.tq_write_rows(q[None, :], BITS, sg, True)
    q_dec = O.tq_decode(qc[0], DIM, BITS, qs[0], qz[0], sg).astype(np.float64)
    corr = np.array([O.qjl_correction(qsb[0], qcm[0], sb[t], c[t], DIM) for t in range(SEQ)])
    np.testing.assert_allclose(logits, k_read.astype(np.float64) @ q_dec + corr, rtol=1e-4,
                               atol=1e-4)
