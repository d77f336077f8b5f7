"""In-tree build of the gfx950 kernel library and the C++ host library.

    python vicold.hybridai_amd/build.py            # both libraries
    python vicold.hybridai_amd/build.py --kernels  # kernel library only

Outputs (git-ignored, shipped with the tree):
    vicold.hybridai_amd/lib/libhai_kernels.so   HIP kernels + C ABI (hai_*)
    vicold.hybridai_amd/lib/libhybridai.so      C++ host: Backend, registries,
                                                verify engine, Generator
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import hashlib
import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
LIB = PKG / "lib"
OBJ = PKG / "_build"
INCLUDE = ROOT / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = os.environ.get("HAI_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off and correctly rounded div/sqrt are part of the numerics
# contract (bit-identical to the CPU oracle); packed FP32 is disabled.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", f"-I{INCLUDE}", f"-I{CSRC}",
]
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++20", "-Wall", "-Wextra", "-Wno-unused-parameter",
             f"-I{INCLUDE}", f"-I{HOST}"]

KERNEL_SOURCES = ["hai_runtime.hip", "hai_gemm.hip", "hai_gemm_fp8.hip", "hai_gemm_mfma.hip", "hai_norm.hip", "hai_attention.hip",
                  "hai_deltanet.hip", "hai_deltanet_prefill.hip", "hai_argmax.hip"]


MANIFEST = LIB / "build_manifest.json"


def kernel_inputs() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))


def host_inputs() -> list[Path]:
    return (sorted(HOST.glob("*.cc")) + sorted(HOST.glob("*.h")) + sorted(HOST.glob("*.inc"))
            + sorted(HOST.glob("refabi/*")) + sorted(INCLUDE.glob("*.h")))


def source_digest(paths) -> str:
    """sha256 over the names and bytes of the sources a library is built from."""
    h = hashlib.sha256()
    for p in paths:
        h.update(str(p.relative_to(ROOT)).encode())
        h.update(p.read_bytes())
    return h.hexdigest()


def _record(lib: str, digest: str) -> None:
    m = json.loads(MANIFEST.read_text()) if MANIFEST.exists() else {}
    m[lib] = digest
    tmp = MANIFEST.with_suffix(".tmp")
    tmp.write_text(json.dumps(m, indent=1) + "\n")
    os.replace(tmp, MANIFEST)


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[-1]}")
    return r


def build_kernels(jobs: int = 8) -> Path:
    OBJ.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    digest = source_digest(kernel_inputs())  # before compiling: an edit during the build leaves it stale
    objs = []
    cmds = []
    for src in KERNEL_SOURCES:
        obj = OBJ / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    out = LIB / "libhai_kernels.so"
    tmp = LIB / "libhai_kernels.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    _record(out.name, digest)
    return out


def build_host(jobs: int = 8) -> Path | None:
    # host sources plus the standalone registries of the Backend ABI (refabi/)
    srcs = sorted(HOST.glob("*.cc")) + sorted(HOST.glob("refabi/*.cc")) if HOST.exists() else []
    if not srcs:
        return None
    OBJ.mkdir(exist_ok=True)
    digest = source_digest(host_inputs())
    objs = []
    cmds = []
    for src in srcs:
        obj = OBJ / (src.stem + ".host.o")
        objs.append(obj)
        cmds.append([CXX, *CXX_FLAGS, "-c", str(src), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    out = LIB / "libhybridai.so"
    tmp = LIB / "libhybridai.so.tmp"
    _run([CXX, "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), f"-L{LIB}", "-lhai_kernels",
          "-Wl,-rpath,$ORIGIN", "-lpthread"])
    os.replace(tmp, out)
    _record(out.name, digest)
    return out


def build(kernels_only: bool = False) -> None:
    build_kernels()
    if not kernels_only:
        build_host()


def clean() -> None:
    shutil.rmtree(OBJ, ignore_errors=True)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--kernels", action="store_true")
    ap.add_argument("--clean", action="store_true")
    a = ap.parse_args()
    if a.clean:
        clean()
    build(kernels_only=a.kernels)
    print("built", LIB)
