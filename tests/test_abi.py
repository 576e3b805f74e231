"""The C ABI library builds, loads and exports every symbol the headers
declare (no GPU work is issued here), and its host-side helpers agree with
the oracle."""
import ctypes
import os
import re

import numpy as np

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in ("tenzo.h", "tenzo_hip.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        names |= set(re.findall(r"TENZO(?:_HIP)?_API\s+[\w\s\*]+?\b(tenzo_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    from tenzo_amd import _lib
    L = _lib.load()
    declared = declared_symbols()
    assert len(declared) > 40
    missing = [n for n in sorted(declared) if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(_lib.exported_symbols()) == declared
    assert not _lib.missing_symbols()


def test_version_and_error_strings():
    from tenzo_amd import _lib
    L = _lib.load()
    assert b"gfx950" in L.tenzo_hip_version()
    assert L.tenzo_get_version().startswith(b"1.0.0")
    L.tenzo_hip_last_error()


def test_rope_table_host_helper_matches_oracle():
    from tenzo_amd import _lib
    L = _lib.load()
    for theta in (10000.0, 500000.0):
        cs = np.empty((50, 128), np.float32)
        L.tenzo_hip_rope_table(theta, 128, 4070, 50, ctypes.c_void_p(cs.ctypes.data))
        for p in range(0, 50, 7):
            np.testing.assert_array_equal(cs[p], oracle.rope_table(theta, 4070 + p))


def test_packed_sizes():
    from tenzo_amd import _lib
    L = _lib.load()
    assert L.tenzo_hip_tl1_packed_bytes(6912, 2560) == 6912 * 2560 // 4
    assert L.tenzo_hip_tl1_packed_bytes(64, 66) == 2 * 1024
    assert L.tenzo_hip_i8_packed_bytes(128256, 2560) == 128256 * 2560
    assert L.tenzo_hip_i8_packed_bytes(65, 32) == 2 * 2 * 1024


def test_default_config_matches_reference_defaults():
    from tenzo_amd import engine
    cfg = engine.default_config()
    assert (cfg.hidden_size, cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.num_layers,
            cfg.ffn_dim, cfg.vocab_size, cfg.max_seq_len) == (2560, 20, 5, 128, 30, 6912,
                                                              128256, 8192)
    assert cfg.kv_mode == b"int8_fused"


REFERENCE = "/root/reference"


def test_reference_callers_link_against_the_library(tmp_path):
    """The reference's own SDK callers (examples/basic_inference.cpp and the
    CLI src/main_inference.cpp, which also needs its CPU profiler source)
    compile against include/ (tenzo.hpp, tenzo.h) and link against
    libtenzo_hip.so unchanged; every engine symbol they import is ours.
    Link only, nothing is run. Skipped where the reference checkout is absent."""
    import pytest
    import subprocess
    if not os.path.isdir(os.path.join(REFERENCE, "examples")):
        pytest.skip("reference checkout not present")
    lib = os.path.join(ROOT, "tenzo_amd")
    for name, srcs in (("basic_inference", ["examples/basic_inference.cpp"]),
                       ("main_inference", ["src/main_inference.cpp",
                                           "src/runtime/MicroarchProfiler.cpp"])):
        exe = str(tmp_path / name)
        subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"),
                        "-I", os.path.join(REFERENCE, "src")] +
                       [os.path.join(REFERENCE, s) for s in srcs] +
                       ["-L", lib, "-ltenzo_hip", "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib",
                        "-o", exe], check=True, timeout=300)
        undef = subprocess.run(["nm", "-D", "--undefined-only", exe], capture_output=True,
                               text=True, check=True).stdout
        imported = {ln.split()[-1] for ln in undef.splitlines() if " tenzo_" in ln}
        assert imported and imported <= declared_symbols(), imported - declared_symbols()
