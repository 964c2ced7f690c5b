"""Oracle pins for LowRankKeyDecomposer (onnx-rt/src/kv_compression.rs:420-690)
and CompressedKVCache's low-rank K state (:840-852, read_k :862-889).

Two kinds of check:
* the reference's own unit tests (kv_compression.rs:1312-1482, :1591-1611,
  :1883-1948), restated with the same inputs and bounds;
* closed forms for well-scaled inputs, where sqrt_approx (ten Newton steps
  from x) is exact to f32 rounding and power iteration with a singular-value
  gap converges in ten rounds: the factors equal numpy's SVD (up to sign),
  a rank-1 matrix is reproduced, an update's coefficient is row . Vt, and
  the 512th write re-decomposes the reconstruction.
On badly scaled inputs (squared norms far above 1e4) the reference's
sqrt_approx has not converged after ten steps, so its factors are far from
the SVD; the reference's tests only bound those results, and so do these.
"""
import numpy as np
import pytest

import oracle as O


def l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - np.asarray(b, np.float64)))


def test_reference_error_decreases_with_rank():
    m = np.add.outer(np.arange(16), np.arange(8)).astype(np.float32)
    e = [l2(m, O.LowRankK(m, r).reconstruct()) for r in (1, 2, 4)]
    assert e[1] <= e[0] + 1e-3 and e[2] <= e[1] + 1e-3


def test_reference_rank1_matrix():
    u = np.arange(1, 9, dtype=np.float32)
    v = np.arange(1, 5, dtype=np.float32) * 0.5
    m = np.outer(u, v).astype(np.float32)
    rec = O.LowRankK(m, 1).reconstruct()
    assert l2(m, rec) / (np.linalg.norm(m) + 1e-10) < 0.6


def test_reference_incremental_update():
    m = (np.arange(32, dtype=np.float32) * 0.1).reshape(4, 8)
    lr = O.LowRankK(m, 4, capacity=5)
    assert lr.rows == 4
    lr.update(np.arange(8, dtype=np.float32) * 0.5)
    assert lr.rows == 5 and lr.factors()[0].size == 5 * lr.rank


def test_reference_empty_matrix():
    lr = O.LowRankK(np.zeros((0, 8), np.float32), 4)
    assert lr.rows == 0 and lr.rank == 4 and lr.reconstruct().size == 0


def test_reference_full_rank_diagonal():
    m = np.diag(np.arange(1, 5, dtype=np.float32))
    rec = O.LowRankK(m, 4).reconstruct()
    assert l2(m, rec) / (np.linalg.norm(m) + 1e-10) < 0.01


def test_reference_single_row():
    row = np.arange(1, 9, dtype=np.float32)[None]
    lr = O.LowRankK(row, 4)
    assert lr.rows == 1 and lr.rank == 1
    assert l2(row, lr.reconstruct()) < 1.0


def test_reference_incremental_preserves_cols():
    lr = O.LowRankK(np.arange(16, dtype=np.float32)[None], 4, capacity=11)
    for r in range(10):
        lr.update((np.arange(16) + r).astype(np.float32) * 0.1)
    assert lr.rows == 11 and lr.cols == 16


def test_reference_update_with_zero_row():
    lr = O.LowRankK(np.arange(16, dtype=np.float32).reshape(2, 8), 2, capacity=3)
    lr.update(np.zeros(8, np.float32))
    assert lr.rows == 3
    assert np.all(lr.factors()[0][2] == 0.0)


def test_reference_cache_lowrank_reads():
    """cache_with_lowrank (:1591-1611) and integration_lowrank_improves_k_accuracy
    (:1883-1948): read_k through the low-rank state has the right size and a
    relative error below 2 on an approximately rank-2 K."""
    k8 = np.array([[(i + p) * 0.1 for i in range(16)] for p in range(8)], np.float32)
    assert O.tq_lowrank_rows(k8, 4).reconstruct().shape == (8, 16)
    dim = seq = 16
    b1 = np.arange(dim, dtype=np.float32) * 0.1
    b2 = (dim - np.arange(dim)).astype(np.float32) * 0.05
    k = np.stack([np.float32(p * 0.3) * b1 + np.float32((seq - p) * 0.2) * b2
                  for p in range(seq)]).astype(np.float32)
    lr = O.tq_lowrank_rows(k, 4)
    assert lr.rank == 1
    assert l2(k, lr.reconstruct()) / (np.linalg.norm(k) + 1e-6) < 2.0


def _scaled_matrix(rng, m, n, sig):
    u, _ = np.linalg.qr(rng.standard_normal((m, len(sig))))
    v, _ = np.linalg.qr(rng.standard_normal((n, len(sig))))
    return (u * np.asarray(sig)) @ v.T


@pytest.mark.parametrize("m,n", [(16, 8), (40, 64), (5, 128)])
def test_factors_equal_the_svd_when_well_scaled(m, n):
    rng = np.random.default_rng(m * n)
    a = _scaled_matrix(rng, m, n, [1.0, 0.3, 0.08]).astype(np.float32)
    lr = O.LowRankK(a, 3)
    us, vt = lr.factors()
    U, S, Vt = np.linalg.svd(a.astype(np.float64), full_matrices=False)
    for r in range(3):
        sgn = np.sign(vt[r] @ Vt[r])
        np.testing.assert_allclose(vt[r], sgn * Vt[r], atol=2e-4)
        np.testing.assert_allclose(us[:, r], sgn * S[r] * U[:, r], atol=2e-4)
    np.testing.assert_allclose(lr.reconstruct(), a, atol=1e-4)


def test_rank1_matrix_reproduced_when_well_scaled():
    rng = np.random.default_rng(7)
    u = rng.uniform(0.5, 1.5, 24) * rng.choice([-1.0, 1.0], 24)
    v = rng.standard_normal(32)
    v /= np.linalg.norm(v)
    a = np.outer(u, v).astype(np.float32)
    lr = O.LowRankK(a, 1)
    np.testing.assert_allclose(lr.reconstruct(), a, atol=2e-6)
    # the first row alone: vt = +-row/|row|, u_s = +-|row|
    one = O.LowRankK(a[:1], 4)
    us, vt = one.factors()
    assert one.rank == 1
    np.testing.assert_allclose(abs(us[0, 0]), np.linalg.norm(a[0]), rtol=1e-5)
    np.testing.assert_allclose(np.abs(vt[0]), np.abs(a[0]) / np.linalg.norm(a[0]), atol=1e-6)


def test_update_coefficient_is_the_projection():
    rng = np.random.default_rng(11)
    a = _scaled_matrix(rng, 6, 16, [1.0, 0.2]).astype(np.float32)
    lr = O.LowRankK(a, 2, capacity=7)
    row = rng.standard_normal(16).astype(np.float32)
    lr.update(row)
    us, vt = lr.factors()
    np.testing.assert_allclose(us[6], vt @ row, rtol=1e-5, atol=1e-6)


def test_zero_first_row_keeps_zero_factors():
    lr = O.LowRankK(np.zeros((1, 8), np.float32), 1, capacity=3)
    us, vt = lr.factors()
    assert lr.rank == 1 and not us.any() and not vt.any()
    # a row of tiny norm ends the same way: sqrt_approx of a tiny sum of
    # squares overestimates it, v shrinks each round, sigma falls below 1e-12
    tiny = O.LowRankK(np.full((1, 8), 1e-4, np.float32), 1)
    assert not tiny.factors()[0].any()
    lr.update(np.ones(8, np.float32))
    assert lr.factors()[0][1, 0] == 0.0


def test_512th_write_redecomposes_the_reconstruction():
    """write_counter reaches 512 at rows = 513: U_S Vt is rebuilt and
    decomposed again. On rank-1 rows (well scaled) the new factors are the
    rank-1 SVD of the old reconstruction, the same matrix to rounding."""
    rng = np.random.default_rng(5)
    v = rng.standard_normal(32)
    v /= np.linalg.norm(v)
    # |c| in [0.2, 0.35]: every sum of squares the iteration normalises stays
    # where ten Newton steps from x have converged
    c = rng.uniform(0.2, 0.35, 600) * rng.choice([-1.0, 1.0], 600)
    k = np.outer(c, v).astype(np.float32)
    lr = O.LowRankK(k[:1], 1, capacity=600)
    for t in range(1, 512):
        lr.update(k[t])
    assert lr.rows == 512 and lr.write_counter == 511
    before = lr.reconstruct()
    vt_old = lr.factors()[1][0]
    lr.update(k[512])
    assert lr.rows == 513 and lr.write_counter == 0
    us, vt = lr.factors()
    full = np.vstack([before, np.outer(k[512] @ vt_old, vt_old)])
    np.testing.assert_allclose(lr.reconstruct()[:512], before, atol=2e-6)
    U, S, Vt = np.linalg.svd(full.astype(np.float64), full_matrices=False)
    sgn = np.sign(vt[0] @ Vt[0])
    np.testing.assert_allclose(vt[0], sgn * Vt[0], atol=1e-5)
    np.testing.assert_allclose(us[:, 0], sgn * S[0] * U[:, 0], atol=1e-5)
    for t in range(513, 600):
        lr.update(k[t])
    np.testing.assert_allclose(lr.reconstruct(), k, atol=1e-5)
