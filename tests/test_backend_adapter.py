"""The MI355X hybridai::Backend ("hip") as the reference's registry hands it
out.  CPU: the driver's registry / fallback checks, a compile of the backend
against the reference's own headers, and the declared ABI (virtual order,
enum values) compared with them.  GPU: every path virtual against the oracle
(tests/backend/backend_parity.cc)."""
import os
import re
import subprocess
from pathlib import Path

import pytest

from _hai import ROOT

DRIVER = ROOT / "tests" / "backend" / "_build" / "backend_parity"
REF_SRC = Path("/root/reference/src")
MIRROR = ROOT / "vicold.hybridai_amd" / "host" / "refabi" / "hybridai_abi.h"


def _build_driver():
    subprocess.run(["make", "-s", "-C", str(ROOT / "tests" / "backend")], check=True, capture_output=True)
    return DRIVER


def _run(args):
    r = subprocess.run([str(_build_driver()), *args], capture_output=True, text=True, timeout=300)
    return r.returncode, r.stdout + r.stderr


def test_registry_and_fallbacks_without_device():
    rc, out = _run(["--cpu"])
    assert rc == 0, out
    assert "0 failed" in out


@pytest.mark.gpu
def test_backend_virtuals_match_oracle():
    rc, out = _run([])
    assert rc == 0, out
    assert "backend (gpu)" in out and "0 failed" in out, out


def _virtuals(text):
    body = text[text.index("class Backend {"):]
    body = body[:body.index("\n};")]
    return re.findall(r"virtual\s+[\w:<>,\s\*&]+?\b(\w+)\s*\(", body)


def _enum(text, name):
    m = re.search(r"enum class " + name + r"\s*:\s*\w+\s*\{([^}]*)\}", text)
    return [e.split("=")[0].strip() for e in m.group(1).split(",") if e.strip() and not e.strip().startswith("//")]


needs_reference = pytest.mark.skipif(not REF_SRC.is_dir(), reason="reference tree not mounted")


@needs_reference
def test_backend_compiles_against_reference_headers():
    cmd = ["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-DHAI_WITH_REFERENCE_TREE", f"-I{REF_SRC}",
           f"-I{ROOT / 'include'}", f"-I{ROOT / 'vicold.hybridai_amd' / 'host'}",
           str(ROOT / "vicold.hybridai_amd" / "host" / "mi355x_backend.cc")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@needs_reference
def test_declared_abi_matches_reference():
    ref = (REF_SRC / "backends" / "interface" / "backend.h").read_text()
    mine = MIRROR.read_text()
    assert _virtuals(mine) == _virtuals(ref)
    for header, enum in (("core/status.h", "StatusCode"), ("core/device.h", "DeviceType"),
                         ("core/dtype.h", "DType"), ("backends/interface/backend.h", "MemoryType")):
        assert _enum(mine, enum) == _enum((REF_SRC / header).read_text(), enum), enum
