"""CPU tests of the C ABI: libflashrt_moe.so loads, exports every entry point include/flashrt_moe.h
declares (and the Python mirror binds exactly those), and the host-only entry points (sizes,
version, argument checks that fail before any device work) behave as documented. No kernel is
launched here."""
from __future__ import annotations

import ctypes as C
import os
import re

import pytest

from flashrt_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions() -> set[str]:
    text = open(os.path.join(ROOT, "include", "flashrt_moe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(frt_[a-z0-9_]+)\s*\(", text))


def test_header_matches_bindings():
    assert header_functions() == set(_lib.SIGNATURES)


def test_library_exports_every_symbol():
    L = _lib.lib()
    for name in header_functions():
        assert hasattr(L, name), name


def test_host_entry_points():
    L = _lib.lib()
    assert L.frt_version().decode().startswith("flashrt")
    assert L.frt_q2_mat_bytes(512, 2048) == 294912
    assert L.frt_q2_expert_bytes(2048, 512) == 884736
    assert L.frt_q2_expert_bytes(2560, 640) == 1382400
    assert L.frt_moe_q2_workspace_bytes(2048, 10, 2048, 512, 512) > 0
    assert L.frt_moe_dispatch_workspace_bytes(2048, 10, 512) > 0


def test_argument_errors_before_device_work():
    """Shape and null-pointer errors are reported with a status and a message, as the reference's
    std::runtime_error would be, without touching a device."""
    L = _lib.lib()
    rc = L.frt_moe_route_topk(None, None, 1, 512, 10, None, None, None, None, 1 << 30)
    assert rc != 0 and L.frt_last_error()
    rc = L.frt_moe_route_topk(None, None, 1, 512, 0, None, None, None, None, 1 << 30)
    assert rc != 0
    with pytest.raises(_lib.FrtError):
        _lib.check(L.frt_moe_q2_run(None, 0, 512, 2048, 512, None, None, 16, 10, None, None, 0, None, 1, 0))


def test_q2_repack_matches_reference_fixture():
    """The product's host repack (frt_q2_repack) reproduces the reference's compiled repack on the
    golden blocks bit for bit (tests/golden/q2_format.npz, 8 rows x 4096), and repack_expert places
    gate | up | down back to back (quant/q2_0/q2_0.cpp:64-80); bad shapes are refused."""
    import numpy as np
    import flashrt_amd as F
    g = np.load(os.path.join(ROOT, "tests", "golden", "q2_format.npz"))
    assert np.array_equal(F.q2_repack(g["repack_in"], 8, 4096), g["repack_out"])
    rng = np.random.default_rng(1)
    n, ff = 256, 128
    mats = [rng.integers(0, 256, r * (c // 64) * 18, dtype=np.uint8) for r, c in ((ff, n), (ff, n), (n, ff))]
    blob = F.q2_repack_expert(*mats, n, ff)
    want = np.concatenate([F.q2_repack(mats[0], ff, n), F.q2_repack(mats[1], ff, n), F.q2_repack(mats[2], n, ff)])
    assert np.array_equal(blob, want)
    with pytest.raises(F.FrtError):
        F.q2_repack(mats[0], ff, 100)


def test_load_experts_reports_io_errors():
    """A missing shard file is an FRT_ERR_IO error with its path in the message (checked before any
    device work)."""
    import flashrt_amd as F
    arena = F._lib.FrtArena(C.c_void_p(1), F.expert_bytes(1024, 256), 0, 1, 1)
    a = F.ExpertArena(arena)
    with pytest.raises(F.FrtError) as e:
        F.load_experts(["/nonexistent/model.gguf"], [(0, 0)] * 3, 1024, 256, a, threads=1)
    assert e.value.code == -5 and "/nonexistent/model.gguf" in str(e.value)


def test_product_does_not_use_the_oracle():
    """The product package never imports or loads anything under oracle/."""
    pkg = os.path.join(ROOT, "flashrt_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"(import\s+oracle|from\s+oracle|liboracle|libfrref|oracle/)", text), \
                    os.path.join(dirpath, f)


def test_cpp_mirror_host():
    """The C++ mirror (include/flashrt_moe.hpp) compiles into a client and maps status codes to
    std::runtime_error (built by `make -C flashrt_amd/csrc`)."""
    import subprocess
    exe = os.path.join(ROOT, "tests", "cpp", "_build", "test_shim")
    assert os.path.exists(exe), "build first: make -C flashrt_amd/csrc"
    r = subprocess.run([exe, "--host"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "all passed" in r.stdout, r.stdout + r.stderr
