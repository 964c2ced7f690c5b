"""Writes the golden fixtures of the quantised-cache GQA path:
tests/golden/<case>.npz and tests/golden/manifest.json.

    python tests/golden/make_golden.py

For each case of golden_data.CASES the manifest records the generator (seed,
streams), the RoPE steps as hex floats, the sha256 of every input, of the whole
cache contents and of every stored array. A fixture stores the expected
attention output rows and the last 64 tokens of codes and quantisation
parameters of every (sequence, kv head), all computed by the oracle. Fixtures
are test data: inputs and expected outputs, at most 64 KiB each.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

import golden_data as G  # noqa: E402


def main() -> None:
    manifest = {}
    for name, c in G.CASES.items():
        cs, sn = G.rope_steps(c["d"], c["theta"])
        manifest[name] = {
            "file": f"{name}.npz",
            "case": c,
            "seed": G.SEED_BASE + c["cfg"],
            "streams": {"k": "10 + append index", "v": "20 + append index", "q": 30},
            "rope": {"theta": c["theta"], "rows": G.total_tokens(name),
                     "cos_step_hex": [float(x).hex() for x in cs],
                     "sin_step_hex": [float(x).hex() for x in sn]},
        }
    for name in G.CASES:
        m = manifest[name]
        appends, (ks, vs), q = G.inputs(name)
        cos, sin = G.rope_for(name, manifest)
        ins = {"cos": cos, "sin": sin, "q": q, "step_k": ks, "step_v": vs}
        for i, (k, v) in enumerate(appends):
            ins[f"append{i}_k"], ins[f"append{i}_v"] = k, v
        m["inputs_sha256"] = {k: G.sha256(v) for k, v in ins.items()}
        arrays, out = G.oracle_run(name, manifest)
        m["cache_sha256"] = {k: G.sha256(v) for k, v in arrays.items()}
        m["out_rows"] = G.out_rows(name).tolist()
        fixture = {"out": out, **G.tails(arrays, G.total_tokens(name))}
        m["fixture_sha256"] = {k: G.sha256(v) for k, v in fixture.items()}
        path = os.path.join(HERE, m["file"])
        np.savez(path, **fixture)
        print(f"{name}: {os.path.getsize(path)} bytes")
    with open(G.MANIFEST, "w") as f:
        json.dump(manifest, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
