"""The committed golden fixtures (tests/golden/) against the oracle.

The fixtures freeze, for one small case per workload, the oracle's cache
contents (sha256 of every code and quantisation parameter, and the last 64
tokens stored) and attention output. Here the inputs are regenerated from the
manifest's seeds and the oracle must reproduce every fixture bit for bit; the
GPU tests compare the HIP path with the same fixtures.
"""
import os

import numpy as np
import pytest

from golden import golden_data as G

NAMES = sorted(G.CASES)


@pytest.fixture(scope="module")
def manifest():
    return G.load_manifest()


def test_manifest_lists_every_case_and_sizes(manifest):
    assert sorted(manifest) == NAMES
    for name in NAMES:
        path = os.path.join(G.HERE, manifest[name]["file"])
        assert os.path.getsize(path) <= G.MAX_FIXTURE_BYTES, name
        fx = G.load_fixture(name, manifest)
        assert sorted(fx) == sorted(manifest[name]["fixture_sha256"])
        for k, v in fx.items():
            assert G.sha256(v) == manifest[name]["fixture_sha256"][k], f"{name}:{k}"


def test_generators_are_exact():
    # Irwin-Hall normals: every value is a multiple of 2^-17 within +-6
    z = G.normals(G.SEED_BASE, 99, (4096,)).astype(np.float64)
    assert np.all(np.abs(z) <= 6.0)
    assert np.all(z * 2.0**17 == np.round(z * 2.0**17))
    assert abs(z.mean()) < 0.1 and abs(z.var() - 1.0) < 0.1
    # bf16 rounding: ties to even on hand-picked bit patterns
    x = np.array([0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F807FFF], np.uint32).view(np.float32)
    want = np.array([0x3F800000, 0x3F820000, 0x3F810000, 0x3F800000], np.uint32)
    np.testing.assert_array_equal(G.to_bf16_f32(x).view(np.uint32), want)
    # the recurrence tables stay on the unit circle
    c, s = G.rope_tables_from_steps(4096, *G.rope_steps(128, 5e5))
    assert np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1).max() < 1e-6
    np.testing.assert_array_equal(c[0], 1.0)
    np.testing.assert_array_equal(s[0], 0.0)


@pytest.mark.parametrize("name", NAMES)
def test_inputs_regenerate(manifest, name):
    appends, (ks, vs), q = G.inputs(name)
    cos, sin = G.rope_for(name, manifest)
    want = manifest[name]["inputs_sha256"]
    got = {"cos": cos, "sin": sin, "q": q, "step_k": ks, "step_v": vs}
    for i, (k, v) in enumerate(appends):
        got[f"append{i}_k"], got[f"append{i}_v"] = k, v
    assert sorted(got) == sorted(want)
    for k, v in got.items():
        assert G.sha256(v) == want[k], f"{name}: input {k} does not regenerate"


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(manifest, name):
    arrays, out = G.oracle_run(name, manifest)
    m = manifest[name]
    for k, v in arrays.items():
        assert G.sha256(v) == m["cache_sha256"][k], f"{name}: cache {k}"
    fx = G.load_fixture(name, manifest)
    np.testing.assert_array_equal(out.view(np.uint32), fx["out"].view(np.uint32))
    for k, v in G.tails(arrays, G.total_tokens(name)).items():
        np.testing.assert_array_equal(v, fx[k], err_msg=f"{name}: {k}")
    assert np.isfinite(out).all()
