"""Test helpers: load the product package (directory name contains a dot) and
the CPU oracle, and convert between float32 and bf16 bit patterns."""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_package():
    name = "hybridai_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = ROOT / "vicold.hybridai_amd"
    spec = importlib.util.spec_from_file_location(name, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


hai = load_package()
from oracle import oracle as orc  # noqa: E402  (test infrastructure)


def rand_bf16(rng, shape, scale=1.0):
    """Random values already representable in bf16: (float32 values, bits)."""
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    bits = hai.bf16_bits(x)
    return hai.bf16_to_f32(bits).reshape(shape), bits.reshape(shape)


def gpu_available() -> bool:
    """True when the machine exposes an AMD GPU (/dev/kfd).  Deliberately
    independent of the product library, so a GPU box with a missing or
    broken build fails the GPU tests instead of skipping them."""
    import os
    return os.path.exists("/dev/kfd")


def assert_bits_equal(got_bits, want_f32, what=""):
    want_bits = hai.bf16_bits(np.asarray(want_f32, dtype=np.float32)).reshape(-1)
    got = np.asarray(got_bits, dtype=np.uint16).reshape(-1)
    bad = np.nonzero(got != want_bits)[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(
            f"{what}: {bad.size}/{got.size} bf16 mismatches; first at {i}: got "
            f"{hai.bf16_to_f32(got[i:i+1])[0]!r} want {hai.bf16_to_f32(want_bits[i:i+1])[0]!r}")
