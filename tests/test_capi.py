"""C ABI checks that need no GPU: the library loads, exports exactly the entry
points include/sai_hip.h declares, and its host-only functions behave (default
scale, null-handle rejection, no-device init failure)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import oracle as O
import smallaios_amd as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sai_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sai_[a-z0-9_]+)\s*\(", text)))


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", S.LIB_PATH], check=True,
                         stdout=subprocess.PIPE, text=True).stdout
    return sorted({l.split()[-1] for l in out.splitlines() if " T " in l and "sai_" in l})


def test_library_exports_every_declared_entry_point():
    decl = declared_functions()
    assert len(decl) >= 20
    exp = exported_symbols()
    missing = [f for f in decl if f not in exp]
    assert not missing, f"declared but not exported: {missing}"
    extra = [f for f in exp if f not in decl]
    assert not extra, f"exported but not declared: {extra}"
    lib = S.lib()
    for f in decl:
        getattr(lib, f)
    assert set(S.EXPORTS) <= set(decl)


def test_library_exports_only_the_abi():
    out = subprocess.run(["nm", "-D", "--defined-only", S.LIB_PATH], check=True,
                         stdout=subprocess.PIPE, text=True).stdout
    text_syms = [l.split()[-1] for l in out.splitlines() if " T " in l]
    assert all(s.startswith("sai_") or s.startswith("_") for s in text_syms), text_syms


@pytest.mark.parametrize("d", [2, 4, 64, 128, 256])
def test_default_scale_matches_oracle(d):
    assert np.float32(S.default_scale(d)) == np.float32(O.default_scale(d))


def test_null_handles_are_rejected():
    L = S.lib()
    assert L.sai_init(0, None) == -7
    assert L.sai_kvcache_create(None, None, None) == -7
    assert L.sai_kv_append(None, None, 0, None, None, 1, 1, 1, None, None, 0, 0, 0, None) == -7
    assert L.sai_gqa_decode(None, None, 0, None, 1, 1, 1, None, None, 0, 0, 0, 0, 0.0, 0, None,
                            1, None) == -7
    assert L.sai_gqa_prefill(None, None, 0, None, 1, 1, 1, 1, None, None, 0, 0, 0, 0, 0.0, 0,
                             None, 16, None) == -7
    assert L.sai_last_decode_launches(None) == 0
    assert L.sai_kvcache_set_layer_window(None, None, 0, 4) == -7
    assert L.sai_kvcache_advance(None, None, None) == -7
    assert L.sai_last_error(None) == b""
    L.sai_destroy(None)
    L.sai_kvcache_destroy(None)


def test_init_without_a_device_fails_cleanly():
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is visible")
    except ImportError:
        pass
    h = C.c_void_p()
    assert S.lib().sai_init(0, C.byref(h)) == -4
    assert not h.value


def test_header_compiles_as_c():
    src = '#include "sai_hip.h"\nint main(void){ sai_kvcache_desc d = {0}; (void)d; return 0; }\n'
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-x", "c", "-fsyntax-only",
                        "-I", os.path.join(ROOT, "include"), "-"], input=src, text=True,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    assert r.returncode == 0, r.stdout
