"""The allocation-free GQA verify entry point (hai_gqa_verify_noalloc_bf16)
against the workspace entry point it shares its kernels with
(hai_gqa_verify_bf16): bit-identical outputs on two calls in a row, the
second smaller than the first (the fixed device scratch keeps the first
call's partials, which the second must not read), and sizes beyond the
fixed scratch rejected before anything is launched."""
import numpy as np
import pytest

from _hai import hai, rand_bf16

pytestmark = pytest.mark.gpu


def _kern():
    return hai.kernels()


def _inputs(rng, B, T, nq, nkv, D, lens):
    cap = int(max(lens)) + T + 5
    q = rand_bf16(rng, (B * T, nq, D))[1]
    g = rand_bf16(rng, (B * T, nq, D))[1]
    kc = rand_bf16(rng, (B, cap, nkv, D))[1]
    vc = rand_bf16(rng, (B, cap, nkv, D))[1]
    bufs = [hai.DeviceBuffer.from_array(a) for a in (q, g, kc, vc, np.array(lens, np.int32))]
    return cap, bufs


@pytest.mark.parametrize("shapes", [
    [(1, 4, 24, 4, 256, [4092]), (1, 2, 24, 4, 256, [1030])],   # C2 shape, then a C3 verify
    [(2, 3, 8, 2, 128, [700, 333]), (1, 1, 4, 2, 64, [40])],
])
def test_noalloc_equals_workspace_entry(shapes):
    rng = np.random.default_rng(11)
    k = _kern()
    for B, T, nq, nkv, D, lens in shapes:
        cap, (dq, dg, dk, dv, dl) = _inputs(rng, B, T, nq, nkv, D, lens)
        n = B * T * nq * D * 2
        want, got = hai.DeviceBuffer(n), hai.DeviceBuffer(n)
        ws = hai.DeviceBuffer(k.hai_gqa_scratch_bytes(B, T, nq, D, cap))
        hai.check(k.hai_gqa_verify_bf16(want.ptr, dq.ptr, dg.ptr, dk.ptr, dv.ptr, cap, ws.ptr, B, T, nq, nkv, D,
                                        dl.ptr, T, cap, None), "workspace entry")
        hai.check(k.hai_gqa_verify_noalloc_bf16(got.ptr, dq.ptr, dg.ptr, dk.ptr, dv.ptr, cap, B, T, nq, nkv, D,
                                                dl.ptr, T, cap, None), "allocation-free entry")
        assert np.array_equal(got.download(np.uint16), want.download(np.uint16)), (B, T, nq, D, lens)


def test_noalloc_rejects_work_beyond_its_scratch():
    """A call whose partials exceed the fixed 16 MiB is an argument error
    (nothing is launched; every operand is a real, correctly sized buffer)."""
    k = _kern()
    B, T, nq, nkv, D = 1, 4, 24, 4, 256
    cap = 16384  # 4 x 24 x 256 chunks x 258 floats = 25 MiB of partials
    assert k.hai_gqa_scratch_bytes(B, T, nq, D, cap) > (16 << 20)
    q = hai.DeviceBuffer(B * T * nq * D * 2)
    kc = hai.DeviceBuffer(B * cap * nkv * D * 2)
    vc = hai.DeviceBuffer(B * cap * nkv * D * 2)
    out = hai.DeviceBuffer(B * T * nq * D * 2)
    rc = k.hai_gqa_verify_noalloc_bf16(out.ptr, q.ptr, None, kc.ptr, vc.ptr, cap, B, T, nq, nkv, D, None, cap, cap,
                                       None)
    assert rc == hai.ERR_INVALID
    assert "16 MiB" in k.hai_last_error().decode()
