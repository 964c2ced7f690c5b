"""Builds libsai_hip.so (gfx950 only) in-tree with hipcc, then the C++ host
library libsai_gqa_host.so over it with g++.

Each .hip source is compiled to an object with its own flags, then linked into
one shared library that exports only the C ABI of include/sai_hip.h. The host
library (host/gqa_host.cpp) holds no device code.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsai_hip.so")
HOST_LIB = os.path.join(HERE, "libsai_gqa_host.so")
PROBE_LIB = os.path.join(HERE, "libsai_read_probe.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
CXX = os.environ.get("CXX", "g++")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-fvisibility=hidden",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-Wall", "-Wno-unused-function",
    # packed FP32 VALU ops are kept out of the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# per-source extra flags: the append kernel must round every f32 op on its own
EXTRA = {
    "kv_append.hip": ["-ffp-contract=off"],
    "sai_capi.hip": ["-ffp-contract=off"],
    "rotary.hip": ["-ffp-contract=off"],
    "tq_cache.hip": ["-ffp-contract=off"],
}
SOURCES = ["kv_append.hip", "gqa_decode.hip", "gqa_decode_int4.hip", "gqa_prefill.hip",
           "rotary.hip", "copy_rows.hip", "tq_cache.hip", "sai_capi.hip"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        cmd = [HIPCC, *COMMON, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    for cmd, pr in procs:
        out, _ = pr.communicate()
        out = "\n".join(l for l in out.splitlines()
                        if "packed-fp32-ops' is not a recognized feature" not in l)
        if pr.returncode != 0:
            raise RuntimeError(f"hipcc failed: {' '.join(cmd)}\n{out}")
        if verbose and out.strip():
            print(out)
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    build_host()
    build_probe()
    return LIB


def build_probe() -> str:
    """libsai_read_probe.so: the streaming-read ceiling the bench reports."""
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC, *COMMON, "-shared", os.path.join(CSRC, "read_probe.hip"), "-o", tmp])
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build_host() -> str:
    """libsai_gqa_host.so: the C++ mirror of the reference's GPU dispatch API."""
    tmp = HOST_LIB + ".tmp"
    _run([CXX, "-std=c++17", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-Wall", "-Wextra",
          "-D__HIP_PLATFORM_AMD__", "-I", INCLUDE, "-I", "/opt/rocm/include",
          os.path.join(HERE, "host", "gqa_host.cpp"), os.path.join(HERE, "host", "gqa_session.cpp"),
          os.path.join(HERE, "host", "kv_compression.cpp"), "-o", tmp,
          "-L", HERE, "-lsai_hip", "-L", "/opt/rocm/lib", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
