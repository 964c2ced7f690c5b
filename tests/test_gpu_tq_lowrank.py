"""The TurboQuant cache's optional low-rank K (KVCacheConfig::kv_lowrank_k,
LowRankKeyDecomposer, onnx-rt/src/kv_compression.rs:451-690) on the GPU,
against the oracle's restatement.

CompressedKVCache::write_kv (:840-852) decomposes each head's first K row
alone and appends the later rows with update, re-decomposing at every 512th
write. The device state (U_S per row and Vt, rank 1) is compared bit for bit
with oracle.tq_lowrank_rows fed the same rows in the same order, across
passes that cross the re-decompositions at rows 513 and 1025, and read_k's
reconstruction bit for bit with 0 + U_S Vt."""
import numpy as np
import pytest

import oracle as O
import smallaios_amd as S
from _gpu_util import log

pytestmark = pytest.mark.gpu
SEED = 0x5EED0123


@pytest.fixture(scope="module")
def rt():
    import torch
    assert torch.cuda.is_available()
    r = S.Runtime(0)
    yield r
    r.close()


def to_dev(x, bf16):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.to(torch.bfloat16) if bf16 else t).cuda()


def host_vals(x, bf16):
    if not bf16:
        return x
    return O.bf16_bits_to_f32(O.f32_to_bf16_bits(x)).reshape(x.shape)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def k_rows(rng, n, d, kind):
    """K rows: 'normal' (unit entries), 'lowrank' (two directions plus a little
    noise, entries ~0.1 so the iteration's norms stay where sqrt_approx has
    converged)."""
    if kind == "normal":
        return rng.standard_normal((n, d)).astype(np.float32)
    b1, b2 = rng.standard_normal(d), rng.standard_normal(d)
    b1 /= np.linalg.norm(b1)
    b2 /= np.linalg.norm(b2)
    c = rng.uniform(0.2, 0.35, (n, 1)) * rng.choice([-1.0, 1.0], (n, 1))
    return (c * b1 + 0.05 * c * b2 + 0.002 * rng.standard_normal((n, d))).astype(np.float32)


@pytest.mark.parametrize("d,bits,kind", [(128, 4, "normal"), (64, 3, "lowrank"),
                                         (256, 8, "lowrank"), (128, 4, "lowrank")])
def test_lowrank_state_bit_exact(rt, d, bits, kind):
    """Passes of 700 (f32), 330 (bf16) and 3 x 1 rows (write, write_attend,
    write) over 2 sequences x 2 kv heads, two layers; the first pass crosses
    row 513, the second row 1025."""
    log(f"lowrank d={d} bits={bits} {kind}")
    import torch
    B, H, L = 2, 2, 2
    rng = np.random.default_rng(d * 7 + bits)
    cache = S.TqCache(rt, L, H, d, bits, True, B, 1100, seed=SEED, lowrank_k=4)
    fed = {(l, b, h): [] for l in range(L) for b in range(B) for h in range(H)}
    passes = [(700, False, "write"), (330, True, "write"), (1, False, "write"),
              (1, True, "write_attend"), (1, False, "write")]
    for s_new, bf16, how in passes:
        for layer in range(L):
            k = np.stack([np.stack([k_rows(rng, s_new, d, kind) for _ in range(H)], 1)
                          for _ in range(B)]).reshape(B, s_new, H * d)
            v = rng.standard_normal((B, s_new, H * d)).astype(np.float32)
            kd, vd = to_dev(k, bf16), to_dev(v, bf16)
            if how == "write":
                cache.write(layer, kd, vd, B, s_new)
            else:
                q = to_dev(rng.standard_normal((B, 1, 2 * H * d)).astype(np.float32), False)
                out = torch.zeros((B, 1, 2 * H * d), dtype=torch.float32, device="cuda")
                cache.write_attend(layer, q, kd, vd, out, B, 2 * H)
            kv = host_vals(k, bf16).reshape(B, s_new, H, d)
            for b in range(B):
                for h in range(H):
                    fed[(layer, b, h)].append(kv[b, :, h])
        cache.advance()
    torch.cuda.synchronize()
    n = sum(p[0] for p in passes)
    for (layer, b, h), parts in fed.items():
        rows = np.concatenate(parts)
        lr = O.tq_lowrank_rows(rows, 4)
        us, vt = cache.read_lowrank(layer, b, h, 0, n)
        want_us, want_vt = lr.factors()
        assert lr.rank == 1
        assert same_bits(us, want_us[:, 0]), (layer, b, h, np.flatnonzero(us != want_us[:, 0])[:5])
        assert same_bits(vt, want_vt[0]), (layer, b, h)
        if b == 1 and h == 1:
            kk, _ = cache.read(layer, b, h, 1020, 12)
            assert same_bits(kk, lr.reconstruct()[1020:1032]), (layer, b, h)
    ref, _ = cache.memory_bytes()
    per_row = 2 * ((d * bits + 7) // 8 + 25) + 2 * ((d + 63) // 64 * 8 + 12)
    lowrank = L * H * B * (n * 4 + d * 4 + 32)
    assert ref == n * B * L * H * per_row + lowrank
    cache.close()


def test_lowrank_guards(rt):
    import torch
    cache = S.TqCache(rt, 1, 1, 64, 4, False, 1, 64, lowrank_k=0)  # Some(0) = Some(1)
    k = torch.randn(1, 2, 64, device="cuda")
    cache.write(0, k, k, 1, 2)
    with pytest.raises(S.SaiError) as e:
        cache.write(0, k, k, 1, 2)
    assert e.value.kind == "Unsupported"
    with pytest.raises(S.SaiError) as e:
        cache.set_lengths([0])
    assert e.value.kind == "Unsupported"
    cache.advance()
    cache.write(0, k, k, 1, 2)
    cache.advance()
    us, vt = cache.read_lowrank(0, 0, 0, 0, 4)
    assert us.shape == (4,) and vt.shape == (64,)
    cache.reset()
    cache.write(0, k, k, 1, 2)  # a fresh first row after reset
    cache.advance()
    plain = S.TqCache(rt, 1, 1, 64, 4, False, 1, 64)
    with pytest.raises(S.SaiError) as e:
        plain.read_lowrank(0, 0, 0, 0, 1)
    assert e.value.kind == "Unsupported"
    plain.close()
    cache.close()
