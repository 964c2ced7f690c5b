"""The C++ host mirror of the reference's GPU dispatch API
(smallaios_amd/host/gqa_host.hpp), exercised through its test binary
tests/cpp/test_gqa_host (built by __graft_entry__.build()).

The CPU case covers attribute parsing, gqa_validate's messages
(onnx-rt/src/ops/microsoft.rs:933-984) and the error types. The GPU case runs,
in one child process, the restated reference cache tests
(onnx-rt/tests/test_cuda.rs:1124-1375), the first-token GQA tests
(test_cuda.rs:3426-3525), dispatch_gqa's error contract, multi-layer
prefill/decode sessions (global and sliding-window layers, local_window_size)
checked against the oracle (outputs within 2e-3 abs + 1e-2 rel, cache contents
bit-exact), the RotaryEmbedding op and dispatcher (bit-exact), the CPU
attention ops with explicit past/present (present bit-exact), and
Gemma-shaped graphs run through GpuSession (gqa_session.hpp), one of them at
Gemma 3 4B's head_dim 256, and the TurboQuant cache's C++ mirror
(kv_compression.hpp) against the oracle (read_v and the low-rank read_k
bit-exact, attention within tolerance).
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_gqa_host")


def _run(args, timeout):
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/test_gqa_host is not built: run __graft_entry__.build() first")
    print(f"[host-mirror] {' '.join(args)}", flush=True)
    r = subprocess.run([BIN, *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=timeout)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout
    assert "FAIL" not in r.stdout


def test_host_mirror_cpu():
    _run(["--cpu"], 60)


@pytest.mark.gpu
def test_host_mirror_gpu():
    _run(["--gpu"], 110)
