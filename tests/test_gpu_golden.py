"""The HIP path against the committed golden fixtures (tests/golden/).

Inputs regenerate from the manifest's seeds; the cache built by the HIP append
(and, per case, the separate decode step, the fused append + decode step or the
prefill chunk) must hold exactly the fixture's codes and parameters (sha256 of
the whole cache, stored tail equal) and produce the fixture's output within
2e-3 abs + 1e-2 rel.
"""
import numpy as np
import pytest

from _gpu_util import assert_close, dev, log
from golden import golden_data as G

import smallaios_amd as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    r = S.Runtime(0)
    yield r
    r.close()


@pytest.mark.parametrize("name", sorted(G.CASES))
def test_hip_path_matches_fixture(rt, name):
    import torch
    log(f"golden {name}")
    manifest = G.load_manifest()
    c = G.CASES[name]
    b, hq, hkv, d, new = c["batch"], c["hq"], c["hkv"], c["d"], c["new"]
    total = G.total_tokens(name)
    cos, sin = G.rope_for(name, manifest)
    cos_d, sin_d, rows = dev(cos), dev(sin), cos.shape[0]
    appends, (ks, vs), q = G.inputs(name)
    pages = (total + S.PAGE_TOKENS - 1) // S.PAGE_TOKENS
    quant = S.KV_INT8 if c["quant"] == G.INT8 else S.KV_INT4
    cache = S.KvCache(rt, 1, hkv, d, b * pages, b, pages, quant)
    cache.set_page_table(S.identity_page_table(b, pages))
    kvd = c["kv_dtype"]
    for k, v in appends:
        cache.append(0, dev(k, kvd), dev(v, kvd), b, k.shape[1], cos_d, sin_d, rows)
        cache.advance()
    out = torch.zeros((b, new, hq * d), dtype=torch.float32, device="cuda")
    qd = dev(q, c["q_dtype"])
    if c["step"] == "fused":
        cache.decode_with_cache(0, qd, dev(ks, kvd), dev(vs, kvd), out, b, hq, cos_d, sin_d, rows)
    else:
        cache.append(0, dev(ks, kvd), dev(vs, kvd), b, new, cos_d, sin_d, rows)
        if c["step"] == "decode":
            cache.decode(0, qd, out, b, hq, cos_d, sin_d, rows)
        else:
            cache.prefill(0, qd, out, b, new, hq, cos_d, sin_d, rows)
    torch.cuda.synchronize()
    got = out.cpu().numpy()[:, G.out_rows(name)]

    # cache contents, tokens [0, total) of every (sequence, kv head)
    parts = {"k_codes": [], "v_codes": [], "k_params": [], "v_params": []}
    for bi in range(b):
        row = {k: [] for k in parts}
        for h in range(hkv):
            kc, vc, kp, vp = cache.read(0, bi, h, 0, total)
            for k, a in zip(parts, (kc, vc, kp, vp)):
                row[k].append(a)
        for k in parts:
            parts[k].append(np.stack(row[k]))
    arrays = {k: np.stack(v) for k, v in parts.items()}
    fx = G.load_fixture(name, manifest)
    for k, v in G.tails(arrays, total).items():
        np.testing.assert_array_equal(v, fx[k], err_msg=f"{name}: {k}")
    for k, v in arrays.items():
        assert G.sha256(v) == manifest[name]["cache_sha256"][k], f"{name}: cache {k} differs"
    err = assert_close(got, fx["out"], name)
    log(f"  max abs err {err:.2e}")
    cache.close()
