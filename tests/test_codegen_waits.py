"""The skinny GEMM kernels that stage activation rows by global -> LDS copies
wait for those copies with s_waitcnt vmcnt(n), where n is the number of
weight requests issued after the copies: vector-memory loads of a wave
complete in issue order, so the wait retires every copy while n weight
chunks stay in flight.  The wait is only right when exactly n requests sit
between the last copy and the wait in the code the compiler emits (a request
sunk below the wait leaves copies unretired: a race on the staged rows).
This test compiles hai_gemm.hip for gfx950 with the build's flags and checks
that count in every kernel that stages by copies, and that no later wait of
the prologue (its LDS barriers) drains the requests it prefetched.  CPU only
(hipcc cross-compiles)."""
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "vicold.hybridai_amd"))


def _kernels(asm: str):
    lines = asm.split("\n")
    for i, line in enumerate(lines):
        m = re.match(r"^(_Z\S*gemm_bf16\S*kernel\S*):", line)
        if not m:
            continue
        end = next(j for j in range(i, len(lines)) if "s_endpgm" in lines[j])
        yield m.group(1), lines[i:end]


def test_staged_copy_waits_count_the_requests_behind_them(tmp_path):
    import build
    if not Path(build.HIPCC).exists() and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    out = tmp_path / "gemm.s"
    flags = [f for f in build.HIP_FLAGS if f != "-fPIC"]
    subprocess.run([build.HIPCC, *flags, "--cuda-device-only", "-S", str(build.CSRC / "hai_gemm.hip"), "-o", str(out)],
                   check=True, capture_output=True, timeout=600)
    checked = 0
    for name, body in _kernels(out.read_text()):
        copies = [k for k, l in enumerate(body) if "global_load_lds" in l]
        if not copies:
            continue
        last = copies[-1]
        wait = next(k for k in range(last, len(body)) if "s_waitcnt" in body[k] and "vmcnt(" in body[k])
        n = int(re.search(r"vmcnt\((\d+)\)", body[wait]).group(1))
        issued = sum(1 for k in range(last + 1, wait) if "buffer_load" in body[k] or
                     ("global_load" in body[k] and "lds" not in body[k]))
        assert issued == n, f"{name}: {issued} requests between the copies and s_waitcnt vmcnt({n})"
        # the prologue's block barriers (LDS data only) must not wait for the
        # prefetched requests: the next vector-memory wait still leaves some
        # of them in flight
        nxt = next((k for k in range(wait + 1, len(body)) if "s_waitcnt" in body[k] and "vmcnt(" in body[k]), None)
        if nxt is not None:
            m = int(re.search(r"vmcnt\((\d+)\)", body[nxt]).group(1))
            assert m > 0, f"{name}: the prologue waits for every prefetched request ({body[nxt].strip()})"
        checked += 1
    assert checked >= 4, f"only {checked} staging kernels found"


def test_copy_staged_mfma_pipeline_waits(tmp_path):
    """gemm_dma_mfma_kernel (hai_gemm_mfma.hip): every step issues the
    chunk's 6 + 2 MT copies (weights, scales, activations) and then waits
    with s_waitcnt vmcnt(12 + 4 MT) -- the copies of the two chunks behind
    the one it multiplies -- and no other vector-memory wait stands between
    that wait and the step's LDS reads (a vmcnt(0) there would drain the
    pipeline); no scratch memory (spills would put such waits back)."""
    import build
    if not Path(build.HIPCC).exists() and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    out = tmp_path / "mfma.s"
    flags = [f for f in build.HIP_FLAGS if f != "-fPIC"]
    subprocess.run([build.HIPCC, *flags, "--cuda-device-only", "-S", str(build.CSRC / "hai_gemm_mfma.hip"), "-o",
                    str(out)], check=True, capture_output=True, timeout=900)
    lines = out.read_text().split("\n")
    checked = 0
    for i, line in enumerate(lines):
        m = re.match(r"^(_Z\S*gemm_dma_mfma_kernelILi(\d)\S*):", line)
        if not m:
            continue
        mt = int(m.group(2))
        end = next(j for j in range(i, len(lines)) if "s_endpgm" in lines[j])
        body = lines[i:end]
        assert not any("scratch_" in l for l in body), f"{m.group(1)}: scratch memory"
        ahead = 12 + 4 * mt
        waits = [k for k, l in enumerate(body) if re.search(rf"s_waitcnt vmcnt\({ahead}\)", l)]
        assert waits, f"{m.group(1)}: no s_waitcnt vmcnt({ahead})"
        for k in waits:
            start = max(b for b in range(k) if "s_barrier" in body[b])
            copies = sum(1 for b in range(start, k) if "global_load_lds" in body[b])
            other = sum(1 for b in range(start, k) if ("global_load" in body[b] or "buffer_load" in body[b])
                        and "lds" not in body[b])
            assert copies == 6 + 2 * mt and other == 0, f"{m.group(1)}: {copies} copies, {other} loads before the wait"
            read = next(b for b in range(k, len(body)) if "ds_read_b128" in body[b])
            stray = [body[b].strip() for b in range(k + 1, read) if "vmcnt(" in body[b]]
            assert not stray, f"{m.group(1)}: {stray} between the pipeline wait and the reads"
        checked += 1
    assert checked >= 6, f"only {checked} copy-staged kernels found"
